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

Differences, on purpose: no JIT build, lock file or barrier (the library is built
ahead of time); no CPU fallback when the library is missing - the call raises;
the training operator (``for_inference=False``) and the CPU operator are not
part of this library (``NotImplementedError``); the kernels run on torch's
current stream instead of the legacy default stream.
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


def load_wkv_operator(device: str = "cuda", for_inference: bool = False,
                      head_size: int = HEAD_SIZE) -> Callable:
    if device == "cpu":
        raise NotImplementedError(
            "rwkvtune_amd provides the GPU WKV7 path only; there is no CPU operator")
    if device == "cuda":
        if for_inference:
            return load_hip_operator_inference(head_size)
        raise NotImplementedError(
            "the training WKV7 operator (for_inference=False) is not part of this library")
    raise ValueError(f"Unsupported device type: {device}, only 'cpu' or 'cuda' supported")


load_wkv7_operator = load_wkv_operator


def rwkv7_wkv(q, w, k, v, a, b, head_size=HEAD_SIZE, state=None, return_state=False):
    device_type = os.environ.get("RWKV_DEVICE", "auto")
    if device_type == "auto":
        device_type = "cuda" if q.is_cuda else "cpu"
    for_inference = (state is not None) or return_state
    operator = load_wkv_operator(device=device_type, for_inference=for_inference, head_size=head_size)
    return operator(q, w, k, v, a, b, state, return_state)


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
