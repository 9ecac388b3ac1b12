"""CPU restatement of the reference's WKV7 training operator (test
infrastructure; see ``oracle/__init__``).

``train_forward(r, w, k, v, a, b, s0=None, seg=16, dtype=float64)``
    ``rwkvtune/models/rwkv7/operators/cuda/wkv7_cuda.cu:10-54`` (``forward_kernel``):
    per token ``sa = S a`` with the old state, ``S = S diag(exp(-exp(w))) + v k^T +
    sa b^T``, ``y = S r``; returns ``(y, sa, ckpt, S_final)`` where ``ckpt`` holds the
    state after every ``seg``-th token (``:45-51``) and, as this build also stores,
    after the last one.  Inputs ``[B, T, H, N]``; ``s0`` ``[B, H, N, N]`` (the
    infinite-context op's initial state, ``wkv7_infctx_cuda.cu:24-83``).
``train_backward(r, w, k, v, a, b, dy, ckpt, sa, ds_in=None, seg=16)``
    ``wkv7_cuda.cu:56-131`` (``backward_kernel``, "wind backstepping"): walk t =
    T-1 .. 0, reload ``S_t`` from the checkpoint at each segment end, step it back
    with ``S_{t-1} = (S_t - v k^T - sa b^T) / w~`` and carry ``dS`` (``:79-130``);
    ``ds_in`` is the gradient of the final state and the returned ``ds0`` the
    initial state's (``wkv7_infctx_cuda.cu:105-305``).  Returns
    ``(dr, dw, dk, dv, da, db, ds0)``.

Pinning (tests/test_oracle_wkv7_train.py): the forward equals ``wkv7_rowwise``;
every gradient, including the initial state's and the contribution of a final-
state gradient, equals torch autograd through ``wkv7_rowwise`` in float64 (the
backstepping is exact algebra; float64 leaves ~1e-12); the checkpoint layout
and segment reloads are exercised by T not a multiple of 16 and by seg = 1.
"""

from __future__ import annotations

import torch


def train_forward(r, w, k, v, a, b, s0=None, seg: int = 16, dtype=torch.float64):
    r, w, k, v, a, b = (t.to(dtype) for t in (r, w, k, v, a, b))
    B, T, H, N = r.shape
    dec = torch.exp(-torch.exp(w))
    S = torch.zeros(B, H, N, N, dtype=dtype) if s0 is None else s0.to(dtype).clone()
    y = torch.zeros(B, T, H, N, dtype=dtype)
    sa = torch.zeros(B, T, H, N, dtype=dtype)
    nck = (T + seg - 1) // seg
    ckpt = torch.zeros(B, H, nck, N, N, dtype=dtype)
    for t in range(T):
        sat = torch.einsum("bhij,bhj->bhi", S, a[:, t])
        S = S * dec[:, t, :, None, :] + v[:, t, :, :, None] * k[:, t, :, None, :] + sat[..., None] * b[:, t, :, None, :]
        y[:, t] = torch.einsum("bhij,bhj->bhi", S, r[:, t])
        sa[:, t] = sat
        if (t + 1) % seg == 0 or t == T - 1:
            ckpt[:, :, t // seg] = S
    return y, sa, ckpt, S


def train_backward(r, w, k, v, a, b, dy, ckpt, sa, ds_in=None, seg: int = 16, dtype=torch.float64):
    r, w, k, v, a, b, dy, ckpt, sa = (t.to(dtype) for t in (r, w, k, v, a, b, dy, ckpt, sa))
    B, T, H, N = r.shape
    lw = -torch.exp(w)
    dec = torch.exp(lw)
    grads = [torch.zeros(B, T, H, N, dtype=dtype) for _ in range(6)]
    dr, dw, dk, dv, da, db = grads
    dS = torch.zeros(B, H, N, N, dtype=dtype) if ds_in is None else ds_in.to(dtype).clone()
    S = None
    for t in range(T - 1, -1, -1):
        if (t + 1) % seg == 0 or t == T - 1:
            S = ckpt[:, :, t // seg].clone()              # S_t
        rt, kt, vt, at, bt, dyt, sat, wt = (x[:, t] for x in (r, k, v, a, b, dy, sa, dec))
        dr[:, t] = torch.einsum("bhji,bhj->bhi", S, dyt)  # sum_j S_t[j][i] dy_j
        S = (S - vt[..., :, None] * kt[..., None, :] - sat[..., :, None] * bt[..., None, :]) / wt[..., None, :]
        dS = dS + dyt[..., :, None] * rt[..., None, :]    # dS_t
        dw[:, t] = torch.einsum("bhji,bhji->bhi", dS, S) * wt * lw[:, t]
        dk[:, t] = torch.einsum("bhji,bhj->bhi", dS, vt)
        dv[:, t] = torch.einsum("bhij,bhj->bhi", dS, kt)
        dsa = torch.einsum("bhij,bhj->bhi", dS, bt)
        db[:, t] = torch.einsum("bhji,bhj->bhi", dS, sat)
        da[:, t] = torch.einsum("bhji,bhj->bhi", S, dsa)
        dS = dS * wt[..., None, :] + dsa[..., :, None] * at[..., None, :]
    return dr, dw, dk, dv, da, db, dS
