"""WKV7 operators backed by the gfx950 HIP library - the drop-in for
``rwkvtune/models/rwkv7/operators/wkv_loader.py``.

Public surface (same names, arguments and errors as the reference):

``load_wkv_operator(device='cuda', for_inference=True, head_size=64)``
    ``wkv_loader.py:511-546``; the inference operator it returns behaves like
    ``RUN_CUDA_RWKV7S`` (``wkv_loader.py:465-497``):
    ``op(r, w, k, v, a, b, state=None, return_state=False)`` -
    ``ValueError`` when ``state`` is None, ``RuntimeError`` for inputs that are not
    ``[T, C]`` / ``[B, T, C]`` or of an unsupported dtype; ``y`` has ``r``'s dtype and
    shape; ``state`` (float32 ``[B, H, N, N]``) is updated in place and returned.
``load_wkv7_operator``   alias (``operators/__init__.py:20``).
``rwkv7_wkv(q, w, k, v, a, b, head_size=64, state=None, return_state=False)``
    ``wkv_loader.py:550-581``: device from ``RWKV_DEVICE`` or the tensors.

Plus the slot-table entry points the engine uses directly: ``wkv7_decode``
(single token on a resident state pool, rows addressed through ``slot_idx``) and
``wkv7_prefill`` (ragged packed prompts, ``cu_seqlens``).

``load_wkv_operator(device='cuda', for_inference=False)`` / ``load_hip_operator_train``
    the training operator ``RUN_CUDA_RWKV7g(q, w, k, v, a, b)`` of
    ``wkv_loader.py:201-356``: inputs cast to bf16 and viewed ``[B, T, H, 64]``,
    ``T % 16 == 0`` asserted, ``y`` bf16 ``[B, T, C]``, gradients (bf16) for all
    six inputs through ``WindBackstepping`` on ``rwkv7_wkv_train_forward`` /
    ``_backward``.
``rwkv7_wkv_infctx(w, q, k, v, a, b, state=None, scale=1.0)``
    ``operators/wkv_infctx.py:164-210``: ``(y, final_state)`` with gradients for the
    inputs and the initial state, and a final-state gradient flowing in;
    ``load_hip_operator_infctx()`` returns the raw ``forward`` / ``backward`` pair of
    ``wkv7_infctx_op`` (``wkv_loader.py:588-705``).

Differences, on purpose: no JIT build, lock file or barrier (the library is built
ahead of time); no CPU fallback when the library is missing - the call raises;
the CPU operator is not part of this library (``NotImplementedError``); the
kernels run on torch's current stream instead of the legacy default stream; the
infinite-context backward recomputes the forward once (checkpoints every 16
tokens) instead of re-running it from the initial state for every segment.
The reference's loader names (``load_cuda_operator_*``) are aliases here.
"""

from __future__ import annotations

import os
import threading
from typing import Callable

import torch

from . import _lib

HEAD_SIZE = 64

_op_lock = threading.Lock()
_inference_op = None


def _check_inputs(fn, r, w, k, v, a, b):
    if r.ndim not in (2, 3):
        raise RuntimeError(f"Unexpected input shape: {tuple(r.shape)}, expected [T, C] or [B, T, C]")
    for t in (w, k, v, a, b):
        if t.shape != r.shape or t.dtype != r.dtype or t.device != r.device:
            raise RuntimeError(f"{fn}: r, w, k, v, a, b must share shape, dtype and device")
    if r.dtype not in _lib.DTYPE_CODE:
        raise RuntimeError(f"Unsupported dtype for wkv7s operator: {r.dtype}")
    if not r.is_cuda:
        raise RuntimeError(f"{fn}: inputs must be on a GPU device")


def _contig(*ts):
    """Contiguous copies where needed, plus a fresh copy of any tensor whose data
    pointer is not aligned to 4 elements (the kernels read 4 elements at once)."""
    out = []
    for t in ts:
        t = t.contiguous()
        if t.data_ptr() % (4 * t.element_size()):
            t = t.clone()
        out.append(t)
    return out


def _check_out(y, r):
    if y.shape != r.shape or y.dtype != r.dtype or y.device != r.device or not y.is_contiguous():
        raise RuntimeError("y must be a contiguous tensor with r's shape, dtype and device")


def wkv7s_forward(state, r, w, k, v, a, b, head_size: int = HEAD_SIZE):
    """Raw op: ``y = WKV7(state; r, w, k, v, a, b)``, state updated in place.

    ``[T, C]`` inputs are batch 1 (``wkv_loader.py:469-472``).
    """
    _check_inputs("wkv7s_forward", r, w, k, v, a, b)
    if head_size != HEAD_SIZE:
        raise RuntimeError(f"head_size {head_size} not supported (library is built for {HEAD_SIZE})")
    if r.ndim == 2:
        T, C = r.shape
        B = 1
    else:
        B, T, C = r.shape
    H = C // head_size
    if state.dtype != torch.float32 or state.device != r.device:
        raise RuntimeError("state must be a float32 tensor on the inputs' device")
    if state.numel() != B * H * head_size * head_size or not state.is_contiguous():
        raise RuntimeError(f"state must be a contiguous [B={B}, H={H}, {head_size}, {head_size}] tensor")
    r, w, k, v, a, b = _contig(r, w, k, v, a, b)
    y = torch.empty(r.shape, dtype=r.dtype, device=r.device)
    _lib.call("rwkv7s_forward", _lib.dtype_code(r.dtype), B, T, C, H, _lib.ptr(state),
              *(_lib.ptr(t) for t in (r, w, k, v, a, b)), _lib.ptr(y), _lib.stream_of(r))
    return y


def _make_inference_op(head_size: int) -> Callable:
    def RUN_HIP_RWKV7S(r, w, k, v, a, b, state=None, return_state=False):
        if state is None:
            raise ValueError("wkv7s requires state parameter")
        with torch.no_grad():
            y = wkv7s_forward(state, r, w, k, v, a, b, head_size)
        if return_state:
            return y, state
        return y
    return RUN_HIP_RWKV7S


def load_hip_operator_inference(head_size: int = HEAD_SIZE) -> Callable:
    """Counterpart of ``load_cuda_operator_inference`` (``wkv_loader.py:359-504``)."""
    global _inference_op
    if _inference_op is not None:
        return _inference_op
    with _op_lock:
        if _inference_op is None:
            _lib.load()  # fail loudly now if the library is missing
            _inference_op = _make_inference_op(head_size)
    return _inference_op


# ---------------------------------------------------------------------------
# Training operator (wkv_loader.py:201-356) and infinite-context operator
# (operators/wkv_infctx.py, wkv_loader.py:588-705)
# ---------------------------------------------------------------------------

CHUNK_LEN = 16  # wkv_loader.py:263: the standard training op needs T % 16 == 0

_train_op = None
_infctx_op = None


def _train_forward(w, q, k, v, a, b, s0=None, s_out=None):
    """Launch ``rwkv7_wkv_train_forward`` on ``[B, T, H, 64]`` contiguous inputs of
    one dtype; returns ``(y, ckpt, sa)``."""
    B, T, H, N = q.shape
    dev = q.device
    y = torch.empty_like(v)
    nck = (T + CHUNK_LEN - 1) // CHUNK_LEN
    ckpt = torch.empty((B, H, nck, N, N), dtype=torch.float32, device=dev)
    sa = torch.empty((B, T, H, N), dtype=torch.float32, device=dev)
    P = _lib.ptr
    _lib.call("rwkv7_wkv_train_forward", _lib.dtype_code(q.dtype), B, T, H, P(q), P(w), P(k), P(v), P(a), P(b),
              P(y), P(s0), P(s_out), P(ckpt), P(sa), _lib.stream_of(q))
    return y, ckpt, sa


def _train_backward(w, q, k, v, a, b, dy, ckpt, sa, ds_in=None, want_ds0=False):
    B, T, H, N = q.shape
    grads = [torch.empty_like(x) for x in (w, q, k, v, a, b)]
    dw, dq, dk, dv, da, db = grads
    ds0 = torch.empty((B, H, N, N), dtype=torch.float32, device=q.device) if want_ds0 else None
    P = _lib.ptr
    _lib.call("rwkv7_wkv_train_backward", _lib.dtype_code(q.dtype), B, T, H, P(q), P(w), P(k), P(v), P(a), P(b),
              P(dy), P(ckpt), P(sa), P(ds_in), P(dq), P(dw), P(dk), P(dv), P(da), P(db), P(ds0),
              _lib.stream_of(q))
    return dw, dq, dk, dv, da, db, ds0


class WindBackstepping(torch.autograd.Function):
    """``wkv_loader.py:309-334``: forward saves the inputs, the state checkpoints
    and sa; backward returns bf16 gradients of (w, q, k, v, z, b)."""

    @staticmethod
    def forward(ctx, w, q, k, v, z, b):
        B, T, H, C = w.shape
        assert T % CHUNK_LEN == 0, f"Sequence length {T} must be divisible by {CHUNK_LEN}"
        w, q, k, v, z, b = [i.to(torch.bfloat16) if i.dtype != torch.bfloat16 else i
                            for i in [w, q, k, v, z, b]]
        assert all(i.is_contiguous() for i in [w, q, k, v, z, b])
        y, ckpt, sa = _train_forward(w, q, k, v, z, b)
        ctx.save_for_backward(w, q, k, v, z, b, ckpt, sa)
        return y

    @staticmethod
    def backward(ctx, *grad_outputs):
        (dy,) = grad_outputs
        assert dy.dtype == torch.bfloat16
        dy = dy.contiguous()
        w, q, k, v, z, b, ckpt, sa = ctx.saved_tensors
        dw, dq, dk, dv, dz, db, _ = _train_backward(w, q, k, v, z, b, dy, ckpt, sa)
        return dw, dq, dk, dv, dz, db


def _make_train_op(head_size: int) -> Callable:
    def RUN_CUDA_RWKV7g(q, w, k, v, a, b):
        """``wkv_loader.py:336-349``: inputs ``[B, T, H*64]``, output bf16 ``[B, T, H*64]``."""
        B, T, HC = q.shape
        q, w, k, v, a, b = [i.to(torch.bfloat16) if i.dtype != torch.bfloat16 else i for i in [q, w, k, v, a, b]]
        if not q.is_cuda:
            raise RuntimeError("the WKV7 training operator runs on the HIP library only: inputs must be on a GPU")
        q, w, k, v, a, b = [i.view(B, T, HC // head_size, head_size) for i in [q, w, k, v, a, b]]
        y = WindBackstepping.apply(w, q, k, v, a, b)
        return torch.reshape(y, (B, T, HC))
    return RUN_CUDA_RWKV7g


def load_hip_operator_train(head_size: int = HEAD_SIZE) -> Callable:
    """Counterpart of ``load_cuda_operator_train`` (``wkv_loader.py:201-356``)."""
    global _train_op
    if head_size != HEAD_SIZE:
        raise RuntimeError(f"head_size {head_size} not supported (library is built for {HEAD_SIZE})")
    if _train_op is not None:
        return _train_op
    with _op_lock:
        if _train_op is None:
            _lib.load()
            _train_op = _make_train_op(head_size)
    return _train_op


class WKV7InfctxFunction(torch.autograd.Function):
    """``operators/wkv_infctx.py:18-160``: forward saves the inputs and the initial
    state; backward recomputes the forward's checkpoints and runs the backward
    pass with the incoming final-state gradient."""

    @staticmethod
    def forward(ctx, w, q, k, v, a, b, state):
        B, T, H, C = q.shape
        if state is None:
            state = torch.zeros(B, H, C, C, dtype=torch.float32, device=q.device)
        if state.dtype != torch.float32:
            state = state.to(torch.float32)
        state = state.contiguous()
        s = torch.empty_like(state)
        y, _, _ = _train_forward(w, q, k, v, a, b, s0=state, s_out=s)
        ctx.save_for_backward(w, q, k, v, a, b, state)
        return y, s

    @staticmethod
    def backward(ctx, dy, dstate_out):
        w, q, k, v, a, b, s0 = ctx.saved_tensors
        dy = dy.contiguous()
        ds_in = None if dstate_out is None else dstate_out.to(torch.float32).contiguous()
        _, ckpt, sa = _train_forward(w, q, k, v, a, b, s0=s0)
        dw, dq, dk, dv, da, db, ds0 = _train_backward(w, q, k, v, a, b, dy, ckpt, sa, ds_in=ds_in, want_ds0=True)
        return dw, dq, dk, dv, da, db, ds0


def rwkv7_wkv_infctx(w, q, k, v, a, b, state=None, scale: float = 1.0):
    """``operators/wkv_infctx.py:164-210``: ``[B, T, H, 64]`` inputs (cast to q's
    dtype), optional float32 initial state ``[B, H, 64, 64]``; returns
    ``(y, final_state)``."""
    if scale != 1.0:
        q = q * scale
    B, T, H, C = q.shape
    if state is None:
        state = torch.zeros(B, H, C, C, dtype=torch.float32, device=q.device)
    if not q.is_cuda:
        raise RuntimeError("the WKV7 infctx operator runs on the HIP library only: inputs must be on a GPU")
    if q.dtype not in _lib.DTYPE_CODE:
        raise RuntimeError(f"Unsupported dtype for the infctx operator: {q.dtype}")
    dt = q.dtype
    w, k, v, a, b = (x.to(dt).contiguous() for x in (w, k, v, a, b))
    q = q.contiguous()
    return WKV7InfctxFunction.apply(w, q, k, v, a, b, state)


class _InfctxModule:
    """The raw ``forward`` / ``backward`` of ``wkv7_infctx_op``
    (``wkv7_infctx_op.cpp``), in place on caller-owned tensors."""

    @staticmethod
    def forward(w, q, k, v, a, b, s, y):
        """y <- WKV7 from initial state s; s <- final state (float32, in place)."""
        out, _, _ = _train_forward(w, q, k, v, a, b, s0=s, s_out=s)
        y.copy_(out)

    @staticmethod
    def backward(w, q, k, v, a, b, dy, s0, ds_in, dw, dq, dk, dv, da, db, ds):
        ds_in = ds_in if (ds_in is not None and ds_in.numel() > 0) else None
        _, ckpt, sa = _train_forward(w, q, k, v, a, b, s0=s0)
        g = _train_backward(w, q, k, v, a, b, dy.contiguous(), ckpt, sa, ds_in=ds_in, want_ds0=True)
        for dst, src in zip((dw, dq, dk, dv, da, db, ds), g):
            dst.copy_(src)


def load_hip_operator_infctx():
    """Counterpart of ``load_cuda_operator_infctx`` (``wkv_loader.py:588-705``)."""
    global _infctx_op
    if _infctx_op is None:
        with _op_lock:
            if _infctx_op is None:
                _lib.load()
                _infctx_op = _InfctxModule()
    return _infctx_op


def load_wkv_operator(device: str = "cuda", for_inference: bool = False,
                      head_size: int = HEAD_SIZE) -> Callable:
    if device == "cpu":
        raise NotImplementedError(
            "rwkvtune_amd provides the GPU WKV7 path only; there is no CPU operator")
    if device == "cuda":
        if for_inference:
            return load_hip_operator_inference(head_size)
        return load_hip_operator_train(head_size)
    raise ValueError(f"Unsupported device type: {device}, only 'cpu' or 'cuda' supported")


load_wkv7_operator = load_wkv_operator
load_cuda_operator_train = load_hip_operator_train
load_cuda_operator_inference = load_hip_operator_inference
load_cuda_operator_infctx = load_hip_operator_infctx


def rwkv7_wkv(q, w, k, v, a, b, head_size=HEAD_SIZE, state=None, return_state=False):
    device_type = os.environ.get("RWKV_DEVICE", "auto")
    if device_type == "auto":
        device_type = "cuda" if q.is_cuda else "cpu"
    for_inference = (state is not None) or return_state
    operator = load_wkv_operator(device=device_type, for_inference=for_inference, head_size=head_size)
    if for_inference:
        return operator(q, w, k, v, a, b, state, return_state)
    return operator(q, w, k, v, a, b)


# ---------------------------------------------------------------------------
# Slot-table entry points (no reference counterpart at this granularity)
# ---------------------------------------------------------------------------

def wkv7_decode(state_pool, slot_idx, r, w, k, v, a, b, y=None):
    """Single-token WKV7 for ``B`` rows on a resident pool ``[S, H, N, N]``.

    ``r..b`` are ``[B, C]``; row ``i`` uses pool slot ``slot_idx[i]`` (int32 device
    tensor or None for identity); negative slots are skipped.  Returns ``y``.
    """
    _check_inputs("wkv7_decode", r, w, k, v, a, b)
    B, C = r.shape[0], r.shape[-1]
    H = C // HEAD_SIZE
    S = state_pool.shape[0]
    if state_pool.dtype != torch.float32 or tuple(state_pool.shape[1:]) != (H, HEAD_SIZE, HEAD_SIZE) \
            or not state_pool.is_contiguous():
        raise RuntimeError("state_pool must be contiguous float32 [S, H, 64, 64]")
    if slot_idx is not None and (slot_idx.dtype != torch.int32 or slot_idx.numel() != B
                                 or slot_idx.device != r.device):
        raise RuntimeError("slot_idx must be an int32 device tensor with one entry per row")
    if y is None:
        y = torch.empty(r.shape, dtype=r.dtype, device=r.device)
    _check_out(y, r)
    ins = _contig(r, w, k, v, a, b)  # kept alive until the launch is enqueued
    _lib.call("rwkv7_wkv_decode", _lib.dtype_code(r.dtype), B, H, _lib.ptr(state_pool), S,
              _lib.ptr(slot_idx), *(_lib.ptr(t) for t in ins), _lib.ptr(y), _lib.stream_of(r))
    return y


def wkv7_prefill(state_pool, slot_idx, cu_seqlens, r, w, k, v, a, b, y=None, chunk_len: int = 0):
    """Ragged prefill over packed ``[total, C]`` inputs split by ``cu_seqlens``.

    ``cu_seqlens`` and ``slot_idx`` are int32 device tensors (``slot_idx`` may be
    None for identity).  Each sequence starts from its pool slot's state and leaves
    its final state there.  Returns ``y`` (``[total, C]``).  ``chunk_len`` 0, 16,
    32 or 64 runs the chunked matrix-core kernel, 1 the token-serial one; both
    compute the same recurrence.
    """
    _check_inputs("wkv7_prefill", r, w, k, v, a, b)
    total, C = r.shape[0], r.shape[-1]
    H = C // HEAD_SIZE
    nseq = cu_seqlens.numel() - 1
    S = state_pool.shape[0]
    if state_pool.dtype != torch.float32 or tuple(state_pool.shape[1:]) != (H, HEAD_SIZE, HEAD_SIZE) \
            or not state_pool.is_contiguous():
        raise RuntimeError("state_pool must be contiguous float32 [S, H, 64, 64]")
    if cu_seqlens.dtype != torch.int32 or cu_seqlens.device != r.device:
        raise RuntimeError("cu_seqlens must be an int32 device tensor")
    if slot_idx is not None and (slot_idx.dtype != torch.int32 or slot_idx.numel() != nseq
                                 or slot_idx.device != r.device):
        raise RuntimeError("slot_idx must be an int32 device tensor with one entry per sequence")
    if y is None:
        y = torch.empty(r.shape, dtype=r.dtype, device=r.device)
    _check_out(y, r)
    ins = _contig(r, w, k, v, a, b)  # kept alive until the launch is enqueued
    _lib.call("rwkv7_wkv_prefill", _lib.dtype_code(r.dtype), nseq, H, total,
              _lib.ptr(cu_seqlens), _lib.ptr(slot_idx), _lib.ptr(state_pool), S,
              *(_lib.ptr(t) for t in ins), _lib.ptr(y), int(chunk_len), _lib.stream_of(r))
    return y
