"""Pins the WKV7 oracle (CPU only).

Each check is chosen so that a plausible mistake in a restatement fails it:
a swapped a/b, a transposed state (row = key instead of value), a decay applied
on the wrong axis or with the wrong sign, a dropped term, an off-by-one in time.
"""

import math

import pytest
import torch

from oracle import cref
from oracle.wkv7 import wkv7_cpu, wkv7_ragged, wkv7_rowwise
from rwkvtune_amd.workloads import cu_seqlens_of, wkv_inputs, wkv_state


def _rel(x, ref):
    return float((x.double() - ref.double()).norm() / ref.double().norm().clamp_min(1e-300))


def test_hand_2x2_single_step():
    """One step on a 2x2 state computed by hand (N=2, H=1)."""
    S0 = torch.tensor([[[[1.0, 2.0], [3.0, 4.0]]]], dtype=torch.float64)
    dec = torch.tensor([0.5, 0.25], dtype=torch.float64)
    w_raw = torch.log(-torch.log(dec)).view(1, 1, 2)
    a = torch.tensor([1.0, -1.0]).view(1, 1, 2)
    b = torch.tensor([0.5, 2.0]).view(1, 1, 2)
    k = torch.tensor([1.0, 0.0]).view(1, 1, 2)
    v = torch.tensor([2.0, -1.0]).view(1, 1, 2)
    r = torch.tensor([1.0, 1.0]).view(1, 1, 2)
    # sa = S a = [-1, -1]; S' = S*dec + v k^T + sa b^T = [[2, -1.5], [0, -1]]; y = S' r
    S_exp = torch.tensor([[2.0, -1.5], [0.0, -1.0]], dtype=torch.float64)
    y_exp = torch.tensor([0.5, -1.0], dtype=torch.float64)
    for fn in (wkv7_rowwise, lambda *x, **kw: wkv7_cpu(*x, **kw)):
        y, S = fn(r, w_raw, k, v, a, b, head_size=2, state=S0.clone())
        assert torch.allclose(S[0, 0].double(), S_exp, atol=1e-6), S
        assert torch.allclose(y[0, 0].double(), y_exp, atol=1e-6), y
    y, S = cref.wkv7_ref_f64(r, w_raw.float(), k, v, a, b, head_size=2, state=S0)
    assert torch.allclose(S[0, 0], S_exp, atol=1e-6)
    assert torch.allclose(y[0, 0], y_exp, atol=1e-6)


def test_linear_attention_closed_form():
    """a=b=0 and decay 1 (w_raw=-inf): y_t = S0 r_t + sum_{s<=t} v_s (k_s . r_t)."""
    B, T, H, N = 2, 7, 2, 64
    inp = wkv_inputs((B, T), H, N, seed=3, dtype=torch.float32)
    z = torch.zeros_like(inp.r)
    w = torch.full_like(inp.r, -math.inf)
    S0 = wkv_state(B, H, N, seed=4).double()
    y, S = wkv7_rowwise(inp.r, w, inp.k, inp.v, z, z, N, S0)
    r = inp.r.double().view(B, T, H, N).transpose(1, 2)
    k = inp.k.double().view(B, T, H, N).transpose(1, 2)
    v = inp.v.double().view(B, T, H, N).transpose(1, 2)
    att = torch.tril(r @ k.transpose(-1, -2))                 # [B,H,T,T]
    y_cf = att @ v + r @ S0.transpose(-1, -2)                 # [B,H,T,N]
    y_cf = y_cf.transpose(1, 2).reshape(B, T, H * N)
    S_cf = S0 + v.transpose(-1, -2) @ k                       # sum_s v_s k_s^T
    assert _rel(y, y_cf) < 1e-12
    assert _rel(S, S_cf) < 1e-12
    yc, Sc = cref.wkv7_ref_f64(inp.r, w, inp.k, inp.v, z, z, N, S0)
    assert _rel(yc, y_cf) < 1e-12 and _rel(Sc, S_cf) < 1e-12


def test_diagonal_decay_closed_form():
    """a=b=0: S_t = S0 diag(d_t) + sum_s v_s (k_s * d_t/d_s)^T with d_t = prod decay."""
    B, T, H, N = 1, 9, 2, 64
    inp = wkv_inputs((B, T), H, N, seed=5, dtype=torch.float32)
    z = torch.zeros_like(inp.r)
    S0 = wkv_state(B, H, N, seed=6).double()
    y, S = wkv7_rowwise(inp.r, inp.w, inp.k, inp.v, z, z, N, S0)
    lw = -torch.exp(inp.w.double()).view(B, T, H, N).transpose(1, 2)   # [B,H,T,N]
    c = torch.cumsum(lw, dim=2)
    r = inp.r.double().view(B, T, H, N).transpose(1, 2)
    k = inp.k.double().view(B, T, H, N).transpose(1, 2)
    v = inp.v.double().view(B, T, H, N).transpose(1, 2)
    ys = []
    for t in range(T):
        St = S0 * torch.exp(c[:, :, t])[:, :, None, :]
        for s in range(t + 1):
            St = St + v[:, :, s, :, None] * (k[:, :, s] * torch.exp(c[:, :, t] - c[:, :, s]))[:, :, None, :]
        ys.append(torch.einsum("bhij,bhj->bhi", St, r[:, :, t]))
    y_cf = torch.stack(ys, 2).transpose(1, 2).reshape(B, T, H * N)
    assert _rel(y, y_cf) < 1e-12
    assert _rel(S, St) < 1e-12


def test_delta_rule_write():
    """a=-kk, b=kk, k=kk with |kk|=1 and decay 1: the new state maps kk to v exactly.

    S' = S (I - kk kk^T) + v kk^T  =>  S' kk = v.  A transposed state, swapped a/b or
    a sign error in the sa term breaks this.
    """
    B, H, N = 3, 2, 64
    g = torch.Generator().manual_seed(7)
    kk = torch.nn.functional.normalize(torch.randn(B, 1, H, N, generator=g, dtype=torch.float64), dim=-1)
    v = torch.randn(B, 1, H, N, generator=g, dtype=torch.float64)
    S0 = wkv_state(B, H, N, seed=8).double()
    flat = lambda t: t.reshape(B, 1, H * N)
    w = torch.full((B, 1, H * N), -math.inf, dtype=torch.float64)
    r = torch.randn(B, 1, H * N, generator=g, dtype=torch.float64)
    _, S = wkv7_rowwise(r, w, flat(kk), flat(v), flat(-kk), flat(kk), N, S0)
    got = torch.einsum("bhij,bhj->bhi", S, kk[:, 0])
    assert torch.allclose(got, v[:, 0], atol=1e-12)
    _, Sc = cref.wkv7_ref_f64(r.float(), w.float(), flat(kk).float(), flat(v).float(),
                              flat(-kk).float(), flat(kk).float(), N, S0)
    gotc = torch.einsum("bhij,bhj->bhi", Sc, kk[:, 0].float().double())
    assert torch.allclose(gotc, v[:, 0].float().double(), atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_statements_agree(dtype):
    """wkv_cpu-order (fp32), per-row order (fp64) and the C restatement agree."""
    B, T, H, N = 2, 12, 3, 64
    inp = wkv_inputs((B, T), H, N, seed=9, dtype=dtype)
    S0 = wkv_state(B, H, N, seed=10)
    y64, S64 = wkv7_rowwise(*inp.as_tuple(), N, S0)
    yc, Sc = cref.wkv7_ref_f64(*inp.as_tuple(), N, S0)
    assert _rel(yc, y64) < 1e-12 and _rel(Sc, S64) < 1e-12
    y32, S32 = wkv7_cpu(*inp.as_tuple(), N, S0.clone())
    assert _rel(y32, y64) < 1e-5 and _rel(S32, S64) < 1e-5
    # unbatched [T, C] form returns unbatched results (wkv_cpu.py:35-42,71-74)
    y1, S1 = wkv7_cpu(*(t[0] for t in inp.as_tuple()), N, S0[0].clone())
    assert y1.shape == (T, H * N) and S1.shape == (H, N, N)
    assert _rel(y1, y64[0]) < 1e-5


def test_prefill_equals_steps_and_split():
    B, T, H, N = 2, 10, 2, 64
    inp = wkv_inputs((B, T), H, N, seed=11, dtype=torch.float32)
    S0 = wkv_state(B, H, N, seed=12)
    y, S = wkv7_rowwise(*inp.as_tuple(), N, S0)
    St = S0.double()
    ys = []
    for t in range(T):
        yt, St = wkv7_rowwise(*(x[:, t:t + 1] for x in inp.as_tuple()), N, St)
        ys.append(yt)
    assert _rel(torch.cat(ys, 1), y) < 1e-14 and _rel(St, S) < 1e-14
    y1, S1 = wkv7_rowwise(*(x[:, :4] for x in inp.as_tuple()), N, S0)
    y2, S2 = wkv7_rowwise(*(x[:, 4:] for x in inp.as_tuple()), N, S1)
    assert _rel(torch.cat([y1, y2], 1), y) < 1e-14 and _rel(S2, S) < 1e-14


def test_batch_permutation_and_ragged():
    H, N = 2, 64
    lens = [5, 1, 0, 9]
    cu = cu_seqlens_of(lens)
    inp = wkv_inputs((cu[-1],), H, N, seed=13, dtype=torch.bfloat16)
    pool = wkv_state(6, H, N, seed=14)
    slots = [4, 0, 2, 5]
    y, fin = wkv7_ragged(*inp.as_tuple(), cu, states=pool[slots])
    yc, Sc = cref.wkv7_ref_ragged(*inp.as_tuple(), cu, slots, pool)
    assert _rel(yc, y) < 1e-12
    assert _rel(Sc[slots], fin) < 1e-12
    untouched = [1, 3]
    assert torch.equal(Sc[untouched], pool[untouched].double())
    # a sequence's result does not depend on its neighbours
    y3, S3 = wkv7_rowwise(*(x[cu[3]:cu[4]] for x in inp.as_tuple()), N, pool[5])
    assert _rel(y[cu[3]:cu[4]], y3) < 1e-14 and _rel(fin[3], S3) < 1e-14


def test_zero_r_and_decayed_state():
    """r=0 gives y=0; k=v=a=b=0 only decays the state along the key axis."""
    B, T, H, N = 1, 3, 1, 64
    inp = wkv_inputs((B, T), H, N, seed=15, dtype=torch.float32)
    z = torch.zeros_like(inp.r)
    S0 = wkv_state(B, H, N, seed=16)
    y, _ = wkv7_rowwise(z, inp.w, inp.k, inp.v, inp.a, inp.b, N, S0)
    assert torch.count_nonzero(y) == 0
    _, S = wkv7_rowwise(inp.r, inp.w, z, z, z, z, N, S0)
    d = torch.exp(-torch.exp(inp.w.double())).prod(dim=1).view(H, N)   # per key column
    assert torch.allclose(S[0], S0[0].double() * d[:, None, :], rtol=1e-12, atol=0)
