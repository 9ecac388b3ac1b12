"""ctypes binding of the gfx950 HIP library ``lib/librwkv7_hip.so`` (C ABI in
``include/rwkv7_hip.h``).

torch is imported before the library is opened: torch ships its own HIP runtime
(``libamdhip64.so.7``) and the library's dependency on that soname then binds to
the already-loaded runtime, so both share one device context and one set of
streams.  There is no fallback: if the library is missing, every entry point
raises ``HipLibraryMissing``.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "lib", "librwkv7_hip.so")

DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int

# name -> (restype, argtypes); the whole exported surface of rwkv7_hip.h
SIGNATURES = {
    "rwkv7_abi_version": (_I32, []),
    "rwkv7_last_error": (ctypes.c_char_p, []),
    "rwkv7s_forward": (_I32, [_I32, _I64, _I64, _I64, _I64] + [_P] * 8 + [_P]),
    "rwkv7_wkv_decode": (_I32, [_I32, _I64, _I64, _P, _I64, _P] + [_P] * 7 + [_P]),
    "rwkv7_wkv_prefill": (_I32, [_I32, _I64, _I64, _I64, _P, _P, _P, _I64] + [_P] * 7 + [_I32, _P]),
    "rwkv7_wkv_train_ckpt_floats": (_I64, [_I64, _I64, _I64]),
    "rwkv7_wkv_train_forward": (_I32, [_I32, _I64, _I64, _I64] + [_P] * 11 + [_P]),
    "rwkv7_wkv_train_backward": (_I32, [_I32, _I64, _I64, _I64] + [_P] * 17 + [_P]),
    "rwkv7_shift_mix": (_I32, [_I32, _I64, _I64, _P, _P, _I32, _I64, _P, _P, _I64, _P, _P, _P, _P, _P, _P,
                               _I64, _P, _P, _I32, _P, _P, _P]),
    "rwkv7_final_norm": (_I32, [_I32, _I64, _I64, _P, _P, _I32, _I64, _P, _P, _P, _P, _P]),
    "rwkv7_activation": (_I32, [_I32, _I32, _I64, _P, _P]),
    "rwkv7_tmix_prep": (_I32, [_I32, _I64, _I64, _I32] + [_P] * 6 + [_P, _P, _P, _P]),
    "rwkv7_tmix_post": (_I32, [_I32, _I64, _I64] + [_P] * 5 + [_P, _P, _P]),
    "rwkv7_tmix_decode": (_I32, [_I32, _I64, _I64, _I32] + [_P] * 7 + [_P, _P, _P, _I64, _P, _P, _P]),
    "rwkv7_sample": (_I32, [_I32, _I64, _I64, _P, _I64, _I32, _I64, _P, _P, _P, _P, _P, _P, _P,
                            ctypes.c_uint64, _P, _P, _P, _P, _P]),
    "rwkv7_repetition_penalty": (_I32, [_I64, _I64, _P, _I64, ctypes.c_float] + [_P] * 7 + [_P]),
    "rwkv7_rollout_first": (_I32, [_I64, _I64] + [_P] * 8 + [_I64, _I32, _P, _P]),
    "rwkv7_rollout_activate": (_I32, [_I64, _P, _I64, _I64] + [_P] * 8 + [_I64, _I32, _P, _P]),
    "rwkv7_rollout_commit": (_I32, [_I64, _I64, _I64, _I32] + [_P] * 13 + [_I64, _P, _P, _P, _P]),
    "rwkv7_rollout_prepare": (_I32, [_I64, _I64] + [_P] * 20 + [_P]),
    "rwkv7_admit_copy": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64] + [_P] * 6 + [_P]),
    "rwkv7_gemm_decode_workspace": (_I64, [_I64, _I32, _P, _P]),
    "rwkv7_gemm_decode": (_I32, [_I64, _I32] + [_P] * 8 + [_P, _I64, _P]),
    "rwkv7_gemm_decode_noalloc": (_I32, [_I64, _I32] + [_P] * 8 + [_P]),
    "rwkv7_gemm_decode_partial_count": (_I32, [_I64, _I32, _I32]),
    "rwkv7_gemm_decode_partials": (_I32, [_I64, _P, _P, _I64, _I32, _I32, _P, _I64, _P, _P]),
    "rwkv7_gemm_packed_elems": (_I64, [_I32, _I32]),
    "rwkv7_gemm_pack": (_I32, [_P, _I64, _I32, _I32, _P, _P]),
    "rwkv7_head_logits": (_I32, [_I64, _I32, _I32, _P, _I64, _P, _P, _I64, _P]),
    "rwkv7_head_packed_elems": (_I64, [_I32, _I32]),
    "rwkv7_head_pack": (_I32, [_P, _I64, _I32, _I32, _P, _P]),
    "rwkv7_selective_log_softmax": (_I32, [_I32, _I64, _I64, _P, _I64, _P, _P, _P]),
}

_lock = threading.Lock()
_lib = None


class HipLibraryMissing(RuntimeError):
    pass


def load():
    """Open the library once (thread-safe) and declare every signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise HipLibraryMissing(
                f"{LIB_PATH} is not built; run `python -m rwkvtune_amd.build` "
                "(or __graft_entry__.build()) first")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def call(name: str, *args):
    """Call an entry point and raise ``RuntimeError`` with the library's message on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.rwkv7_last_error().decode(errors="replace")
        err = ValueError if rc == 1 else RuntimeError
        raise err(f"{name} failed (code {rc}): {msg}")
    return rc


def ptr(t):
    """Device pointer of a tensor (or None)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def dtype_code(dt: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dt]
    except KeyError:
        raise RuntimeError(f"Unsupported dtype for the WKV7 library: {dt}") from None
