"""CPU restatement of ``RWKV7Model.forward_with_state`` (test infrastructure;
see ``oracle/__init__``).

Follows ``rwkvtune/models/rwkv7/model.py``:
  block            :382-418  (ln0 on layer 0, ln1, time mix, residual, ln2, channel mix, residual)
  time mix         :174-278  (token shift, six lerps, projections, decay/a/v/gate LoRAs,
                              kk normalise, k update, WKV(r, w, k, v, -kk, kk*a),
                              GroupNorm(H, eps 64e-5), bonus, gate, output projection)
  channel mix      :310-343  (shift, lerp, relu(key)^2, value)
  model            :468-497  (embedding, blocks, ln_out, head over every position)
The WKV recurrence is ``oracle.wkv7``: ``wkv7_cpu`` (the reference CPU operator,
``wkv_cpu.py:9-76``) when ``dtype`` is float32, ``wkv7_rowwise`` otherwise
(float64 is the high-precision oracle).  ``dtype=torch.bfloat16`` restates the
reference's bf16 GPU path: every eager op runs on bf16 tensors and rounds its
result to bf16 (the residual stream included, ``model.py:190-278, 310-343,
382-418``), and the WKV op gets bf16 operands - the raw decay ``w`` too - keeps
its state in float32 and returns bf16 ``y`` (``model.py:233-250``,
``wkv7s.cu:22-53``).  Parameters come as a plain
``{name: tensor}`` state dict with the reference's names; all math runs in
``dtype`` on the CPU (the reference runs float32 on CPU, ``pipeline.py:166-175``).

Pinning (tests/test_oracle_model.py): the float32 and float64 statements agree;
prefill(T) equals T single-token steps; batch rows are independent; a layer with
zeroed output projections is the identity on the residual stream; one token
from a zero state gives S = v k^T and a GroupNorm closed form.  Each term of the
layer is then isolated on an otherwise transparent layer (identity projections,
no shift, no LoRA, gate 1) and checked against values known by hand: the decay
exp(-exp(-softplus(-w0) - 0.5)) at w0 = +30, 0, -30 over two tokens; the value
residual at sigmoid = 1 and 0 (v_first taken, own value kept); the delta rule
b = kk * a removing the fraction a of a unit state along kk (a = 1/2, 1/4); the
key update k (1 + (a - 1) k_a) = 3/4 k; the bonus |x|^2 x; the token-shift
direction (mix 1 reads the previous token); relu(x)^2 of the channel mix at
six points and its shift.  Swapping the decay sign, the value-residual
direction, b = kk for kk * a, relu for relu^2, the shift direction, the bonus
axis or the gate's sigmoid placement each fails at least one of these.  The
bf16 statement is pinned by hand-rounded values on the transparent layer: the
decay operand at w0 = 0 is bf16(-bf16(ln 2) - 0.5) = -1.1875 (not -1.1931), and
a = sigmoid(1) reaches the delta rule as 0.73046875 (not 0.7310586); on a random
model it stays within bf16 rounding of the float64 statement but not closer
than the rounding allows, and its WKV state is float32.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .wkv7 import wkv7_cpu, wkv7_rowwise

N = 64


@dataclass
class OracleConfig:
    n_layer: int
    n_embd: int
    vocab_size: int

    @property
    def n_head(self):
        return self.n_embd // N


def config_of(sd) -> OracleConfig:
    L = 1 + max(int(k.split(".")[1]) for k in sd if k.startswith("blocks."))
    V, C = sd["emb.weight"].shape
    return OracleConfig(L, C, V)


def cast_state_dict(sd, dtype):
    return {k: v.detach().to("cpu").to(dtype) for k, v in sd.items()}


def init_state(cfg: OracleConfig, B: int, dtype=torch.float64):
    C, H = cfg.n_embd, cfg.n_head
    return [{"att_x_prev": torch.zeros(B, C, dtype=dtype),
             "att_kv": torch.zeros(B, H, N, N, dtype=dtype),
             "ffn_x_prev": torch.zeros(B, C, dtype=dtype)} for _ in range(cfg.n_layer)]


def _shift(x, x_prev):
    # xx = [x_prev, x[:, :-1]] - x   (model.py:196-201)
    return torch.cat([x_prev.unsqueeze(1), x[:, :-1]], dim=1) - x


def time_mix(sd, i, cfg, x, v_first, x_prev, att_kv, dtype):
    p = f"blocks.{i}.att."
    B, T, C = x.shape
    H = cfg.n_head
    xx = _shift(x, x_prev)
    xr, xw, xk, xv, xa, xg = (x + xx * sd[p + n].reshape(C) for n in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"))
    r = xr @ sd[p + "receptance.weight"].T
    w_lin = torch.tanh(xw @ sd[p + "w1"]) @ sd[p + "w2"]
    k = xk @ sd[p + "key.weight"].T
    v = xv @ sd[p + "value.weight"].T
    if i == 0:
        v_first = v
    else:
        v = v + (v_first - v) * torch.sigmoid(sd[p + "v0"].reshape(C) + (xv @ sd[p + "v1"]) @ sd[p + "v2"])
    a = torch.sigmoid(sd[p + "a0"].reshape(C) + (xa @ sd[p + "a1"]) @ sd[p + "a2"])
    g = torch.sigmoid(xg @ sd[p + "g1"]) @ sd[p + "g2"]
    kk = F.normalize((k * sd[p + "k_k"].reshape(C)).view(B, T, H, N), dim=-1, p=2.0).view(B, T, C)
    k = k * (1 + (a - 1) * sd[p + "k_a"].reshape(C))
    w = -F.softplus(-(sd[p + "w0"].reshape(C) + w_lin)) - 0.5
    if dtype == torch.float32:
        y, S = wkv7_cpu(r, w, k, v, -kk, kk * a, N, att_kv)
    elif dtype == torch.bfloat16:
        # the reference's GPU op: bf16 operands, float32 state, bf16 y
        ops = [t.to(torch.bfloat16) for t in (r, w, k, v, -kk, kk * a)]
        y, S = wkv7_rowwise(*ops, N, att_kv.to(torch.float32), dtype=torch.float32)
        y = y.to(torch.bfloat16)
    else:
        y, S = wkv7_rowwise(r, w, k, v, -kk, kk * a, N, att_kv, dtype=dtype)
    y = F.group_norm(y.reshape(B * T, C).to(dtype), H, sd[p + "ln_x.weight"], sd[p + "ln_x.bias"],
                     eps=64e-5).view(B, T, C)
    bonus = (r.view(B, T, H, N) * k.view(B, T, H, N) * sd[p + "r_k"].reshape(H, N)).sum(-1, keepdim=True)
    y = y + (bonus * v.view(B, T, H, N)).view(B, T, C)
    y = (y * g) @ sd[p + "output.weight"].T
    return y, v_first, x[:, -1], (S if dtype == torch.bfloat16 else S.to(dtype))


def channel_mix(sd, i, x, x_prev):
    p = f"blocks.{i}.ffn."
    C = x.shape[-1]
    xx = _shift(x, x_prev)
    kx = x + xx * sd[p + "x_k"].reshape(C)
    h = torch.relu(kx @ sd[p + "key.weight"].T) ** 2
    return h @ sd[p + "value.weight"].T, x[:, -1]


def _ln(x, sd, name):
    return F.layer_norm(x, (x.shape[-1],), sd[name + ".weight"], sd[name + ".bias"], 1e-5)


def forward_with_state(sd, idx, states=None, dtype=torch.float64, skip_ln0=False, hidden_only=False):
    """``(logits [B, T, V], new_states)`` in ``dtype``; ``sd`` must already be in ``dtype``.

    ``hidden_only``: return the ln_out output ``[B, T, C]`` instead of logits.
    """
    cfg = config_of(sd)
    B, T = idx.shape
    if states is None:
        states = init_state(cfg, B, dtype)
    x = sd["emb.weight"][idx.reshape(-1)].view(B, T, -1)
    v_first = None
    new_states = []
    for i in range(cfg.n_layer):
        st = states[i]
        if i == 0 and not skip_ln0:
            x = _ln(x, sd, "blocks.0.ln0")
        h = _ln(x, sd, f"blocks.{i}.ln1")
        kv_dt = torch.float32 if dtype == torch.bfloat16 else dtype
        att, v_first, ax, kv = time_mix(sd, i, cfg, h, v_first, st["att_x_prev"].to(dtype),
                                        st["att_kv"].to(kv_dt), dtype)
        x = x + att
        h2 = _ln(x, sd, f"blocks.{i}.ln2")
        ffn, fx = channel_mix(sd, i, h2, st["ffn_x_prev"].to(dtype))
        x = x + ffn
        new_states.append({"att_x_prev": ax, "att_kv": kv, "ffn_x_prev": fx})
    x = _ln(x, sd, "ln_out")
    if hidden_only:
        return x, new_states
    return x @ sd["head.weight"].T, new_states


def greedy_generate(sd, prompts, n_new, dtype=torch.float32, max_valid_id=None):
    """Greedy decode of ``n_new`` tokens after each prompt (a [B, T0] tensor):
    prefill the prompts in one call, then one token per step, argmax over the
    logits with ids above ``max_valid_id`` banned (``core.py:66-83, 171-188``).
    Returns ``(tokens [B, n_new] int64, top-2 logit gaps [B, n_new])``."""
    logits, states = forward_with_state(sd, prompts, None, dtype)
    last = logits[:, -1]
    out, gaps = [], []
    for _ in range(n_new):
        l = last.clone()
        if max_valid_id is not None and max_valid_id + 1 < l.shape[-1]:
            l[:, max_valid_id + 1:] = float("-inf")
        top2 = torch.topk(l, 2, dim=-1).values
        gaps.append(top2[:, 0] - top2[:, 1])
        tok = l.argmax(dim=-1)
        out.append(tok)
        logits, states = forward_with_state(sd, tok[:, None], states, dtype)
        last = logits[:, -1]
    return torch.stack(out, 1), torch.stack(gaps, 1)
