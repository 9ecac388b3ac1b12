"""ctypes binding of ``oracle/wkv7_ref.c`` (fp64 C restatement; test infrastructure).

``build()`` compiles it with the committed ``oracle/Makefile`` (gcc only).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libwkv7_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "libwkv7_oracle.so"],
                       check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        build()
        lib = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        lib.wkv7_ref_f64.argtypes = [ctypes.c_int] * 4 + [P] * 8
        lib.wkv7_ref_f64.restype = None
        lib.wkv7_ref_ragged.argtypes = [ctypes.c_int, P, P, ctypes.c_int, ctypes.c_int] + [P] * 8
        lib.wkv7_ref_ragged.restype = None
        _lib = lib
    return _lib


def _f32(x):
    return np.ascontiguousarray(x.detach().to(torch.float32).cpu().numpy())


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def wkv7_ref_f64(r, w, k, v, a, b, head_size=64, state=None):
    """``[B,T,C]`` inputs -> ``(y float64 [B,T,C], state float64 [B,H,N,N])``."""
    lib = _load()
    B, T, C = r.shape
    N = head_size
    H = C // N
    arrs = [_f32(t) for t in (r, w, k, v, a, b)]
    if state is None:
        S = np.zeros((B, H, N, N), dtype=np.float64)
    else:
        S = np.ascontiguousarray(state.detach().to(torch.float64).cpu().numpy()).copy()
    y = np.zeros((B, T, C), dtype=np.float64)
    lib.wkv7_ref_f64(B, T, H, N, _ptr(S), *[_ptr(x) for x in arrs], _ptr(y))
    return torch.from_numpy(y), torch.from_numpy(S)


def wkv7_ref_ragged(r, w, k, v, a, b, cu_seqlens, seq_slot, state_pool, head_size=64):
    """Packed ``[total, C]`` inputs; updates a float64 copy of ``state_pool``."""
    lib = _load()
    total, C = r.shape
    N = head_size
    H = C // N
    arrs = [_f32(t) for t in (r, w, k, v, a, b)]
    cu = np.ascontiguousarray(np.asarray(cu_seqlens, dtype=np.int32))
    nseq = len(cu) - 1
    slot = None if seq_slot is None else np.ascontiguousarray(np.asarray(seq_slot, dtype=np.int32))
    S = np.ascontiguousarray(state_pool.detach().to(torch.float64).cpu().numpy()).copy()
    y = np.zeros((total, C), dtype=np.float64)
    lib.wkv7_ref_ragged(nseq, _ptr(cu), None if slot is None else _ptr(slot), H, N, _ptr(S),
                        *[_ptr(x) for x in arrs], _ptr(y))
    return torch.from_numpy(y), torch.from_numpy(S)
