"""WKV7 recurrence restated on the CPU (test infrastructure; see ``oracle/__init__``).

Two statements of the same recurrence live here:

``wkv7_cpu``       follows ``rwkvtune/models/rwkv7/operators/wkv_cpu.py:9-76``: inputs
                   are upcast to float, the decay is ``exp(-exp(w))`` (``:49``), and per
                   token ``S = S*w + (S@a)@b + v@k; y = S@r`` (``:61-68``) with batched
                   matmuls.  This is the reference's CPU path and the timed CPU baseline.
``wkv7_rowwise``   follows the per-row order of the reference CUDA kernel
                   ``operators/cuda/wkv7s.cu:22-53``: ``sa_i = sum_j a_j S_ij`` first
                   (``:33-38``), then ``S_ij = S_ij w_j + k_j v_i + sa_i b_j`` and
                   ``y_i = sum_j S_ij r_j`` (``:40-48``).  Run in float64 it is the
                   high-precision oracle the HIP kernels are compared with.

State layout (both): ``[B, H, N, N]``, row ``i`` = value index, column ``j`` = key
index (``wkv7s.cu:13``).  Inputs ``[B, T, C]`` or ``[T, C]`` with ``C = H*N``.

Pinning (tests/test_oracle_wkv7.py): the two statements agree with each other and
with the independent C restatement ``oracle/wkv7_ref.c``; closed forms pin the
terms separately - ``a=b=0`` with decay 1 is causal linear attention, ``a=b=0`` is
the diagonal-decay sum, the delta-rule write ``a=-kk, b=kk, k=kk, |kk|=1`` gives
``S_new kk = v`` exactly, and a 2x2 state is checked against hand arithmetic;
invariants - prefill(T) == T single steps, chunk splitting, batch permutation.
"""

from __future__ import annotations

import torch


def _split(x):
    return x if x.ndim == 3 else x.unsqueeze(0)


def wkv7_cpu(r, w, k, v, a, b, head_size: int = 64, state=None):
    """Reference CPU operator semantics (``wkv_cpu.py:9-76``), float32 math.

    Returns ``(y, state)``; ``y`` is float32 with the input's batch layout, the
    state is a new float32 tensor (the input state is not modified, as in the
    reference where ``state.to(float32)`` of a float32 tensor aliases but the
    loop rebinds ``state``).
    """
    had_batch = r.ndim == 3
    r, w, k, v, a, b = (_split(t) for t in (r, w, k, v, a, b))
    B, T, C = r.shape
    N = head_size
    H = C // N
    r = r.reshape(B, T, H, N).float()
    k = k.reshape(B, T, H, N).float()
    v = v.reshape(B, T, H, N).float()
    a = a.reshape(B, T, H, N).float()
    b = b.reshape(B, T, H, N).float()
    w = torch.exp(-torch.exp(w.reshape(B, T, H, N).float()))
    out = torch.zeros((B, T, H, N), dtype=torch.float32)
    if state is None:
        S = torch.zeros((B, H, N, N), dtype=torch.float32)
    else:
        S = (state if state.ndim == 4 else state.unsqueeze(0)).to(torch.float32)
    for t in range(T):
        kk = k[:, t].reshape(B, H, 1, N)
        rr = r[:, t].reshape(B, H, N, 1)
        vv = v[:, t].reshape(B, H, N, 1)
        aa = a[:, t].reshape(B, H, N, 1)
        bb = b[:, t].reshape(B, H, 1, N)
        S = S * w[:, t, :, None, :] + S @ aa @ bb + vv @ kk
        out[:, t] = (S @ rr).reshape(B, H, N)
    out = out.reshape(B, T, C)
    if not had_batch:
        return out[0], S[0]
    return out, S


def wkv7_rowwise(r, w, k, v, a, b, head_size: int = 64, state=None,
                 dtype=torch.float64, decay_floor=None):
    """Per-row order of ``wkv7s.cu:22-53`` in ``dtype`` (float64 by default).

    ``decay_floor``: optional lower bound applied to the log-decay ``-exp(w)``
    before ``exp`` (the HIP prefill kernel bounds it at -10 for range safety;
    passing the same bound lets a test separate that documented clamp from
    arithmetic error).  Returns ``(y, state)`` in ``dtype``.
    """
    had_batch = r.ndim == 3
    r, w, k, v, a, b = (_split(t).to(dtype) for t in (r, w, k, v, a, b))
    B, T, C = r.shape
    N = head_size
    H = C // N
    shp = (B, T, H, N)
    r, w, k, v, a, b = (t.reshape(shp) for t in (r, w, k, v, a, b))
    lw = -torch.exp(w)
    if decay_floor is not None:
        lw = torch.clamp(lw, min=decay_floor)
    dec = torch.exp(lw)
    if state is None:
        S = torch.zeros((B, H, N, N), dtype=dtype)
    else:
        S = (state if state.ndim == 4 else state.unsqueeze(0)).to(dtype).clone()
    y = torch.zeros(shp, dtype=dtype)
    for t in range(T):
        sa = torch.einsum("bhij,bhj->bhi", S, a[:, t])
        S = (S * dec[:, t, :, None, :]
             + v[:, t, :, :, None] * k[:, t, :, None, :]
             + sa[..., None] * b[:, t, :, None, :])
        y[:, t] = torch.einsum("bhij,bhj->bhi", S, r[:, t])
    y = y.reshape(B, T, C)
    if not had_batch:
        return y[0], S[0]
    return y, S


def wkv7_ragged(r, w, k, v, a, b, cu_seqlens, states=None, head_size: int = 64,
                dtype=torch.float64):
    """Ragged prefill: packed ``[total, C]`` inputs split by ``cu_seqlens``.

    Each sequence runs ``wkv7_rowwise`` from its own initial state (zero when
    ``states`` is None; else ``states[s]``).  Returns ``(y [total, C], final
    states [nseq, H, N, N])``.  This is the sequence-by-sequence meaning of one
    ragged prefill call: no sequence sees another's tokens.
    """
    cu = [int(x) for x in cu_seqlens]
    C = r.shape[-1]
    H = C // head_size
    ys = []
    finals = []
    for s in range(len(cu) - 1):
        lo, hi = cu[s], cu[s + 1]
        st = None if states is None else states[s]
        if hi == lo:
            ys.append(torch.zeros((0, C), dtype=dtype))
            finals.append(torch.zeros((H, head_size, head_size), dtype=dtype)
                          if st is None else st.to(dtype).clone())
            continue
        y, S = wkv7_rowwise(r[lo:hi], w[lo:hi], k[lo:hi], v[lo:hi], a[lo:hi], b[lo:hi],
                            head_size, st, dtype)
        ys.append(y)
        finals.append(S)
    return torch.cat(ys, 0), torch.stack(finals, 0)
