"""Pins the CPU model oracle (oracle/model.py) with invariants and closed forms
that do not restate its own formulas."""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import model as om
from rwkvtune_amd.model import RWKV7Config, build_model

N = 64


def tiny_sd(seed=0, L=2, C=256, V=300, dtype=torch.float64):
    cfg = RWKV7Config(n_layer=L, n_embd=C, vocab_size=V, dim_att_lora=32, dim_gate_lora=64, dim_mv_lora=32)
    m = build_model(cfg, dtype=torch.float32, device="cpu", seed=seed)
    return om.cast_state_dict(m.state_dict(), dtype)


def test_init_is_seeded_and_dense():
    a = tiny_sd(1, dtype=torch.float32)
    b = tiny_sd(1, dtype=torch.float32)
    c = tiny_sd(2, dtype=torch.float32)
    assert all(torch.equal(a[k], b[k]) for k in a)
    assert any(not torch.equal(a[k], c[k]) for k in a)
    # the matrices the reference init leaves at zero are dense here
    for k in ("blocks.0.att.output.weight", "blocks.1.ffn.value.weight", "blocks.0.att.w1",
              "blocks.1.att.v1", "blocks.0.att.g1", "blocks.0.att.a1"):
        assert a[k].abs().min() >= 0 and a[k].abs().mean() > 0
    assert "blocks.0.att.v0" not in a and "blocks.1.att.v0" in a


def test_fp32_matches_fp64():
    sd64 = tiny_sd(3)
    sd32 = om.cast_state_dict(sd64, torch.float32)
    g = torch.Generator().manual_seed(0)
    idx = torch.randint(0, 300, (2, 11), generator=g)
    l64, s64 = om.forward_with_state(sd64, idx, dtype=torch.float64)
    l32, s32 = om.forward_with_state(sd32, idx, dtype=torch.float32)
    assert float((l32.double() - l64).norm() / l64.norm()) < 1e-5
    for a, b in zip(s32, s64):
        for k in a:
            assert float((a[k].double() - b[k]).norm() / b[k].norm().clamp_min(1e-30)) < 1e-5


def test_prefill_equals_token_steps():
    sd = tiny_sd(4)
    g = torch.Generator().manual_seed(1)
    idx = torch.randint(0, 300, (2, 7), generator=g)
    lp, sp = om.forward_with_state(sd, idx)
    st = None
    outs = []
    for t in range(7):
        l, st = om.forward_with_state(sd, idx[:, t:t + 1], st)
        outs.append(l[:, 0])
    ls = torch.stack(outs, 1)
    assert torch.allclose(lp, ls, rtol=1e-10, atol=1e-10)
    for a, b in zip(sp, st):
        for k in a:
            assert torch.allclose(a[k], b[k], rtol=1e-10, atol=1e-12)


def test_split_prefill_carries_state():
    sd = tiny_sd(5)
    g = torch.Generator().manual_seed(2)
    idx = torch.randint(0, 300, (1, 13), generator=g)
    l_all, s_all = om.forward_with_state(sd, idx)
    l1, s1 = om.forward_with_state(sd, idx[:, :6])
    l2, s2 = om.forward_with_state(sd, idx[:, 6:], s1)
    assert torch.allclose(torch.cat([l1, l2], 1), l_all, rtol=1e-10, atol=1e-10)


def test_batch_rows_independent():
    sd = tiny_sd(6)
    g = torch.Generator().manual_seed(3)
    idx = torch.randint(0, 300, (3, 5), generator=g)
    l, _ = om.forward_with_state(sd, idx)
    perm = [2, 0, 1]
    lp, _ = om.forward_with_state(sd, idx[perm])
    assert torch.allclose(lp, l[perm], rtol=1e-12, atol=1e-12)


def test_zero_branches_reduce_to_embedding_path():
    """With the output and FFN value projections at zero (the reference's own
    init) every block is the identity on the residual stream, so the logits are
    head(ln_out(ln0(emb[idx]))) - computed here with plain F.layer_norm."""
    sd = tiny_sd(7)
    for k in list(sd):
        if k.endswith("att.output.weight") or k.endswith("ffn.value.weight"):
            sd[k] = torch.zeros_like(sd[k])
    idx = torch.tensor([[5, 17, 3, 250]])
    l, _ = om.forward_with_state(sd, idx)
    x = sd["emb.weight"][idx]
    C = x.shape[-1]
    x = F.layer_norm(x, (C,), sd["blocks.0.ln0.weight"], sd["blocks.0.ln0.bias"], 1e-5)
    x = F.layer_norm(x, (C,), sd["ln_out.weight"], sd["ln_out.bias"], 1e-5)
    assert torch.allclose(l, x @ sd["head.weight"].T, rtol=1e-12, atol=1e-12)


def test_first_token_time_mix_closed_form():
    """From a zero state, one token gives S = v k^T (no decay or delta term can act
    on a zero state), so y_head = v_head * (k_head . r_head) and
    GroupNorm(y_head) = sign(k.r) * GroupNorm-core(v_head) up to the eps term.
    The output projection is made the identity and the gate constant, so the layer
    output is checked against that closed form."""
    sd = tiny_sd(8, L=1)
    C = 256
    H = C // N
    p = "blocks.0.att."
    sd[p + "output.weight"] = torch.eye(C, dtype=torch.float64)
    sd[p + "g1"] = torch.zeros_like(sd[p + "g1"])       # sigmoid(0) = 1/2 ...
    sd[p + "g2"] = torch.full_like(sd[p + "g2"], 2.0 / sd[p + "g2"].shape[0])  # ... g = 1
    sd[p + "ln_x.weight"] = torch.ones(C, dtype=torch.float64)
    sd[p + "ln_x.bias"] = torch.zeros(C, dtype=torch.float64)
    sd[p + "r_k"] = torch.zeros_like(sd[p + "r_k"])     # no bonus term
    cfg = om.config_of(sd)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, 1, C, generator=g, dtype=torch.float64)
    st = om.init_state(cfg, 1)[0]
    y, _, _, S = om.time_mix(sd, 0, cfg, x, None, st["att_x_prev"], st["att_kv"], torch.float64)
    # operands the layer feeds the recurrence (token shift against a zero x_prev)
    xx = -x
    xr = x + xx * sd[p + "x_r"].reshape(C)
    xk = x + xx * sd[p + "x_k"].reshape(C)
    xv = x + xx * sd[p + "x_v"].reshape(C)
    xa = x + xx * sd[p + "x_a"].reshape(C)
    r = (xr @ sd[p + "receptance.weight"].T).view(H, N)
    v = (xv @ sd[p + "value.weight"].T).view(H, N)
    a = torch.sigmoid(sd[p + "a0"].reshape(C) + (xa @ sd[p + "a1"]) @ sd[p + "a2"]).view(H, N)
    k = (xk @ sd[p + "key.weight"].T).view(H, N) * (1 + (a - 1) * sd[p + "k_a"].reshape(H, N))
    kr = (k * r).sum(-1, keepdim=True)
    # state after one token from zero is v k^T per head
    assert torch.allclose(S[0], v[:, :, None] * k[:, None, :], rtol=1e-12, atol=1e-12)
    vc = v - v.mean(-1, keepdim=True)
    var_y = (kr ** 2) * (vc ** 2).mean(-1, keepdim=True)
    expect = kr * vc / torch.sqrt(var_y + 64e-5)
    assert torch.allclose(y.view(H, N), expect, rtol=1e-9, atol=1e-9)


# ---------------------------------------------------------------------------
# Closed forms that each isolate one term of the time mix / channel mix.  The
# layer is first made transparent (identity projections, no token shift in the
# mixes, zero LoRA downs, gate 1, no delta-rule or bonus term, identity
# GroupNorm affine), then one term at a time is switched on at values whose
# result is known by hand.  A slip in that term (a sign, a swapped lerp, a
# dropped square or factor) fails the corresponding test.
# ---------------------------------------------------------------------------

def _transparent(sd, i, C):
    p = f"blocks.{i}.att."
    eye = torch.eye(C, dtype=torch.float64)
    for n in ("receptance", "key", "value", "output"):
        sd[p + n + ".weight"] = eye.clone()
    for n in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"):
        sd[p + n] = torch.zeros_like(sd[p + n])
    for n in ("w1", "a1", "g1") + (("v1",) if i > 0 else ()):
        sd[p + n] = torch.zeros_like(sd[p + n])
    # g = sigmoid(0) @ g2 with every g2 entry 2 / rank: g = 1 on every channel
    sd[p + "g2"] = torch.full_like(sd[p + "g2"], 2.0 / sd[p + "g2"].shape[0])
    for n in ("k_k", "k_a", "r_k", "a0"):
        sd[p + n] = torch.zeros_like(sd[p + n])
    sd[p + "w0"] = torch.full_like(sd[p + "w0"], -30.0)   # decay exp(-exp(-softplus(30) - .5)) = 1 - 6e-14
    sd[p + "ln_x.weight"] = torch.ones(C, dtype=torch.float64)
    sd[p + "ln_x.bias"] = torch.zeros(C, dtype=torch.float64)
    return p


def _run_time_mix(sd, i, x, v_first=None, S0=None):
    cfg = om.config_of(sd)
    B, T, C = x.shape
    st = om.init_state(cfg, B)[i]
    kv = st["att_kv"] if S0 is None else S0
    return om.time_mix(sd, i, cfg, x, v_first, st["att_x_prev"], kv, torch.float64)


def test_decay_softplus_form_closed_form():
    """w = -softplus(-(w0 + w_lora)) - 0.5 with the decay exp(-exp(w)) applied by
    the recurrence (model.py:227, wkv7s.cu:27).  With k_k = 0 (kk = 0: no
    delta-rule term) and w1 = 0 (w_lora = 0), two tokens from a zero state leave
    S = v1 k1^T diag(d) + v2 k2^T, with d known in closed form at three w0:
      w0 = +30:  softplus(-30) ~ 0       -> d = exp(-e^-0.5)          = 0.5452392...
      w0 =   0:  softplus(0) = ln 2      -> d = exp(-e^-0.5 / 2)      = 0.7384031...
      w0 = -30:  softplus(30) ~ 30       -> d = exp(-e^-30.5) ~ 1."""
    sd = tiny_sd(11, L=1)
    C = 256
    p = _transparent(sd, 0, C)
    pattern = torch.tensor([30.0, 0.0, -30.0], dtype=torch.float64)
    sd[p + "w0"] = pattern.repeat(C // 3 + 1)[:C].reshape(sd[p + "w0"].shape)
    d_of = {30.0: math.exp(-math.exp(-0.5)), 0.0: math.exp(-math.exp(-0.5) / 2), -30.0: 1.0}
    assert abs(d_of[30.0] - 0.5452392) < 1e-7 and abs(d_of[0.0] - 0.7384031) < 1e-7
    d = torch.tensor([d_of[float(w)] for w in sd[p + "w0"].reshape(C)], dtype=torch.float64)
    g = torch.Generator().manual_seed(12)
    x = torch.randn(1, 2, C, generator=g, dtype=torch.float64)
    _, _, _, S = _run_time_mix(sd, 0, x)
    H = C // N
    x1, x2, dh = x[0, 0].view(H, N), x[0, 1].view(H, N), d.view(H, N)
    expect = x1[:, :, None] * (x1 * dh)[:, None, :] + x2[:, :, None] * x2[:, None, :]
    assert torch.allclose(S[0], expect, rtol=1e-11, atol=1e-11)


def test_value_residual_at_sigmoid_saturation():
    """v <- v + (v_first - v) * sigmoid(v0 + v_lora) on layers > 0
    (model.py:215-218): v0 = +40 (sigmoid = 1) takes v_first, v0 = -40
    (sigmoid = 0) keeps the layer's own value.  One token from a zero state
    gives S = v k^T, so row i of each head's state is v_i times k."""
    sd = tiny_sd(13, L=2)
    C = 256
    H = C // N
    p = _transparent(sd, 1, C)
    v0 = torch.tensor([40.0 if (c // N) % 2 == 0 else -40.0 for c in range(C)], dtype=torch.float64)
    sd[p + "v0"] = v0.reshape(sd[p + "v0"].shape)
    g = torch.Generator().manual_seed(14)
    x = torch.randn(1, 1, C, generator=g, dtype=torch.float64)
    u = torch.randn(1, 1, C, generator=g, dtype=torch.float64)   # v_first from layer 0
    _, vf, _, S = _run_time_mix(sd, 1, x, v_first=u)
    assert vf is u
    v_expect = torch.where(v0 > 0, u[0, 0], x[0, 0]).view(H, N)
    k = x[0, 0].view(H, N)
    assert torch.allclose(S[0], v_expect[:, :, None] * k[:, None, :], rtol=1e-12, atol=1e-12)


def test_layer0_value_becomes_v_first():
    sd = tiny_sd(15, L=2)
    C = 256
    _transparent(sd, 0, C)
    g = torch.Generator().manual_seed(16)
    x = torch.randn(1, 3, C, generator=g, dtype=torch.float64)
    _, vf, _, _ = _run_time_mix(sd, 0, x)
    assert torch.allclose(vf, x, rtol=0, atol=0)   # value projection = identity, no shift


def test_delta_rule_uses_kk_times_a():
    """The WKV call is WKV(r, w, k, v, -kk, kk*a) (model.py:246-247).  With the
    value projection at zero (v = 0), a1 = 0 (a = sigmoid(a0)), decay 1, k_k = 1
    and a token whose key is e_0 in every head (kk = e_0), one step from S0 = I
    gives S1 = I - a_0 e_0 e_0^T: the delta rule removes the fraction a of the
    state along kk.  Heads take a0 = 0 (a = 1/2) and a0 = ln(1/3) (a = 1/4):
    S1[0, 0] = 1/2 and 3/4; every other entry stays that of I."""
    sd = tiny_sd(17, L=1)
    C = 256
    H = C // N
    p = _transparent(sd, 0, C)
    sd[p + "value.weight"] = torch.zeros(C, C, dtype=torch.float64)
    sd[p + "k_k"] = torch.ones_like(sd[p + "k_k"])
    a0 = torch.tensor([0.0 if (c // N) % 2 == 0 else math.log(1.0 / 3.0) for c in range(C)], dtype=torch.float64)
    sd[p + "a0"] = a0.reshape(sd[p + "a0"].shape)
    x = torch.zeros(1, 1, C, dtype=torch.float64)
    x[0, 0, ::N] = 3.0
    S0 = torch.eye(N, dtype=torch.float64).expand(1, H, N, N).clone()
    _, _, _, S = _run_time_mix(sd, 0, x, S0=S0)
    expect = S0.clone()
    for h in range(H):
        expect[0, h, 0, 0] = 0.5 if h % 2 == 0 else 0.75
    assert torch.allclose(S, expect, rtol=0, atol=1e-12)


def test_key_update_by_a():
    """k <- k * (1 + (a - 1) * k_a) (model.py:225): a = 1/2 (a0 = 0), k_a = 1/2
    scales the key by 3/4, so one token from a zero state gives S = (3/4) v k^T."""
    sd = tiny_sd(18, L=1)
    C = 256
    H = C // N
    p = _transparent(sd, 0, C)
    sd[p + "k_a"] = torch.full_like(sd[p + "k_a"], 0.5)
    g = torch.Generator().manual_seed(19)
    x = torch.randn(1, 1, C, generator=g, dtype=torch.float64)
    _, _, _, S = _run_time_mix(sd, 0, x)
    xv = x[0, 0].view(H, N)
    assert torch.allclose(S[0], 0.75 * xv[:, :, None] * xv[:, None, :], rtol=1e-12, atol=1e-12)


def test_bonus_term():
    """out += (sum_head r * k * r_k) * v (model.py:267-268): with the GroupNorm
    affine at zero only the bonus reaches the output.  r, k and v are three
    different diagonal scalings of x (r = e_r x, k = e_k x, v = e_v x) and r_k = 1,
    so out_head = (sum_head e_r e_k x^2) e_v x.  The three factors are not
    parallel, so multiplying the sum by k or r, or summing r * v, gives another
    vector."""
    sd = tiny_sd(20, L=1)
    C = 256
    H = C // N
    p = _transparent(sd, 0, C)
    g = torch.Generator().manual_seed(21)
    e = {n: 0.5 + torch.rand(C, generator=g, dtype=torch.float64) for n in ("receptance", "key", "value")}
    for n, d in e.items():
        sd[p + n + ".weight"] = torch.diag(d)
    sd[p + "r_k"] = torch.ones_like(sd[p + "r_k"])
    sd[p + "ln_x.weight"] = torch.zeros(C, dtype=torch.float64)
    x = torch.randn(1, 1, C, generator=g, dtype=torch.float64)
    y, _, _, _ = _run_time_mix(sd, 0, x)
    xh = x[0, 0].view(H, N)
    er, ek, ev = (e[n].view(H, N) for n in ("receptance", "key", "value"))
    expect = (er * ek * xh * xh).sum(-1, keepdim=True) * (ev * xh)
    assert torch.allclose(y[0, 0].view(H, N), expect, rtol=1e-12, atol=1e-12)
    # the wrong factor is far from it
    wrong = (er * ek * xh * xh).sum(-1, keepdim=True) * (ek * xh)
    assert not torch.allclose(wrong, expect, rtol=1e-3, atol=1e-3)


def test_token_shift_lerp_direction():
    """x_mix = x + (x_prev - x) * mix (model.py:196-208): mix = 1 feeds the
    previous token.  With x_r = 1 and everything else transparent, token 2's
    receptance is token 1, so y_2 = GroupNorm(S_2 x_1) with S_2 = x_1 x_1^T +
    x_2 x_2^T; and mix = 0 (x_r = 0) reads x_2 itself."""
    sd = tiny_sd(22, L=1)
    C = 256
    H = C // N
    p = _transparent(sd, 0, C)
    g = torch.Generator().manual_seed(23)
    x = torch.randn(1, 2, C, generator=g, dtype=torch.float64)
    x1, x2 = x[0, 0].view(H, N), x[0, 1].view(H, N)
    S2 = x1[:, :, None] * x1[:, None, :] + x2[:, :, None] * x2[:, None, :]

    def gn(y):
        yc = y - y.mean(-1, keepdim=True)
        return yc / torch.sqrt((yc ** 2).mean(-1, keepdim=True) + 64e-5)

    for mix, rvec in ((1.0, x1), (0.0, x2)):
        sd[p + "x_r"] = torch.full_like(sd[p + "x_r"], mix)
        y, _, x_last, _ = _run_time_mix(sd, 0, x)
        assert torch.allclose(x_last, x[:, -1], rtol=0, atol=0)
        y2 = torch.einsum("hij,hj->hi", S2, rvec)
        assert torch.allclose(y[0, 1].view(H, N), gn(y2), rtol=1e-9, atol=1e-9)


def test_channel_mix_relu_squared_and_shift():
    """FFN = value(relu(key(x + (x_prev - x) * x_k))^2) (model.py:315-338).  With
    key = [I; 0] and value = [I, 0] the output is relu(input)^2 per channel, at
    hand-evaluated points: -2 -> 0, -0.5 -> 0, 0 -> 0, 0.5 -> 0.25, 2 -> 4,
    3 -> 9.  x_k = 0 reads the token, x_k = 1 the previous token."""
    sd = tiny_sd(24, L=1)
    C = 256
    p = "blocks.0.ffn."
    key = torch.zeros(4 * C, C, dtype=torch.float64)
    key[:C] = torch.eye(C, dtype=torch.float64)
    val = torch.zeros(C, 4 * C, dtype=torch.float64)
    val[:, :C] = torch.eye(C, dtype=torch.float64)
    sd[p + "key.weight"], sd[p + "value.weight"] = key, val
    table = {-2.0: 0.0, -0.5: 0.0, 0.0: 0.0, 0.5: 0.25, 2.0: 4.0, 3.0: 9.0}
    pts = torch.tensor(list(table), dtype=torch.float64).repeat(C // 6 + 1)[:C]
    want = torch.tensor([table[float(v)] for v in pts], dtype=torch.float64)
    g = torch.Generator().manual_seed(25)
    other = torch.randn(C, generator=g, dtype=torch.float64)
    # x_k = 0: the token's own value
    sd[p + "x_k"] = torch.zeros_like(sd[p + "x_k"])
    out, last = om.channel_mix(sd, 0, pts.view(1, 1, C), other.view(1, C))
    assert torch.allclose(out[0, 0], want, rtol=0, atol=1e-14)
    assert torch.equal(last[0], pts)
    # x_k = 1: the previous token (x_prev for the first, token 1 for token 2)
    sd[p + "x_k"] = torch.ones_like(sd[p + "x_k"])
    seq = torch.stack([other, pts]).view(1, 2, C)
    out, _ = om.channel_mix(sd, 0, seq, pts.view(1, C))
    assert torch.allclose(out[0, 0], want, rtol=0, atol=1e-14)
    assert torch.allclose(out[0, 1], torch.clamp(other, min=0) ** 2, rtol=1e-14, atol=1e-14)


# ---------------------------------------------------------------------------
# bf16 statement (the reference's bf16 GPU path): hand-rounded values on the
# transparent layer show which operands are rounded to bf16 before the WKV op.
# ---------------------------------------------------------------------------

def _run_time_mix_bf16(sd, i, x, S0=None):
    sd16 = om.cast_state_dict(sd, torch.bfloat16)
    cfg = om.config_of(sd16)
    B, T, C = x.shape
    kv = torch.zeros(B, cfg.n_head, N, N, dtype=torch.float32) if S0 is None else S0.float()
    return om.time_mix(sd16, i, cfg, x.to(torch.bfloat16), None, torch.zeros(B, C, dtype=torch.bfloat16), kv,
                       torch.bfloat16)


def test_bf16_decay_operand_is_rounded():
    """The reference computes w = -softplus(-(w0 + w_lora)) - 0.5 on bf16 tensors
    (model.py:227) and hands the rounded w to the WKV op (wkv7s.cu:27 applies
    exp(-exp(w)) in float).  At w0 = 0: softplus(0) = ln 2 = 0.693147 rounds to
    177/256 = 0.69140625; minus 0.5 gives 1.19140625 = 1.0011000|1b, a tie that
    rounds to even: w = -1.1875 and d = exp(-exp(-1.1875)) = 0.7371361..., not
    the unrounded 0.7384031.  At w0 = +30, w = -0.5 exactly; at -30, w = -30.5.
    Inputs in {+-1, +-2} keep every other product exact, so the float32 state is
    S = x1 x1^T diag(d) + x2 x2^T to float32 rounding."""
    sd = tiny_sd(31, L=1)
    C = 256
    H = C // N
    p = _transparent(sd, 0, C)
    pattern = torch.tensor([30.0, 0.0, -30.0], dtype=torch.float64)
    sd[p + "w0"] = pattern.repeat(C // 3 + 1)[:C].reshape(sd[p + "w0"].shape)
    d_of = {30.0: math.exp(-math.exp(-0.5)), 0.0: math.exp(-math.exp(-1.1875)), -30.0: 1.0}
    assert abs(d_of[0.0] - 0.7371361) < 1e-7
    d = torch.tensor([d_of[float(w)] for w in sd[p + "w0"].reshape(C)], dtype=torch.float64)
    g = torch.Generator().manual_seed(32)
    x = torch.tensor([-2.0, -1.0, 1.0, 2.0], dtype=torch.float64)[torch.randint(0, 4, (1, 2, C), generator=g)]
    y, _, _, S = _run_time_mix_bf16(sd, 0, x)
    assert y.dtype == torch.bfloat16 and S.dtype == torch.float32
    x1, x2, dh = x[0, 0].view(H, N), x[0, 1].view(H, N), d.view(H, N)
    expect = x1[:, :, None] * (x1 * dh)[:, None, :] + x2[:, :, None] * x2[:, None, :]
    assert torch.allclose(S[0].double(), expect, rtol=2e-7, atol=2e-7)


def test_bf16_delta_rule_gets_rounded_a():
    """a = sigmoid(a0 + a_lora) is a bf16 tensor in the reference (model.py:221),
    so b = kk * a reaches the WKV op rounded: at a0 = 1, sigmoid(1) = 0.7310586
    rounds to 187/256 = 0.73046875.  As in the float64 delta-rule test (kk = e_0,
    v = 0, decay 1, S0 = I) one step gives S1[0, 0] = 1 - a = 0.26953125
    exactly, where the unrounded a would give 0.2689414."""
    sd = tiny_sd(33, L=1)
    C = 256
    H = C // N
    p = _transparent(sd, 0, C)
    sd[p + "value.weight"] = torch.zeros(C, C, dtype=torch.float64)
    sd[p + "k_k"] = torch.ones_like(sd[p + "k_k"])
    sd[p + "a0"] = torch.ones_like(sd[p + "a0"])
    x = torch.zeros(1, 1, C, dtype=torch.float64)
    x[0, 0, ::N] = 3.0
    S0 = torch.eye(N, dtype=torch.float64).expand(1, H, N, N).clone()
    _, _, _, S = _run_time_mix_bf16(sd, 0, x, S0=S0)
    expect = S0.clone()
    expect[0, :, 0, 0] = 0.26953125
    assert torch.equal(S.double(), expect)


def test_bf16_statement_within_rounding_of_fp64():
    """On a random two-layer model the bf16 statement's logits and states stay
    within bf16 rounding of the float64 statement on the same (bf16) weights,
    and differ from it by more than float32 arithmetic would: each eager op is
    rounded.  The WKV state it returns is float32 and the logits bf16."""
    sd16 = tiny_sd(34, L=2, dtype=torch.bfloat16)
    sd64 = om.cast_state_dict(sd16, torch.float64)
    idx = torch.randint(0, 300, (2, 9), generator=torch.Generator().manual_seed(35))
    l16, s16 = om.forward_with_state(sd16, idx, dtype=torch.bfloat16)
    l64, s64 = om.forward_with_state(sd64, idx, dtype=torch.float64)
    assert l16.dtype == torch.bfloat16 and s16[0]["att_kv"].dtype == torch.float32

    def rel(a, b):
        return float((a.double() - b).norm() / b.norm())

    assert 1e-4 < rel(l16, l64) < 2e-2
    for l in range(2):
        for k in ("att_x_prev", "att_kv", "ffn_x_prev"):
            assert rel(s16[l][k], s64[l][k]) < 2e-2, (l, k)
