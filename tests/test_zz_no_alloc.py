"""``rwkv7_gemm_decode_noalloc`` (split-K partials in the library's static
scratch, no allocation) against ``rwkv7_gemm_decode`` (caller workspace), both
called through the C ABI: bit-identical outputs on two calls in a row, the
second with a smaller problem set.  (That no valid problem set needs more
scratch than RWKV7_GEMM_SCRATCH_FLOATS is checked on the CPU, test_capi.py.)
"""

import ctypes

import pytest
import torch

from rwkvtune_amd import _lib
from rwkvtune_amd.model import PackedWeight

pytestmark = pytest.mark.gpu

SCRATCH_FLOATS = 1 << 21   # RWKV7_GEMM_SCRATCH_FLOATS in include/rwkv7_hip.h
P = ctypes.c_void_p


def _arrays(M, probs):
    n = len(probs)
    A = (P * n)(*[a.data_ptr() for a, _, _, _ in probs])
    B = (P * n)(*[b.t.data_ptr() for _, b, _, _ in probs])
    C = (P * n)(*[c.data_ptr() for _, _, c, _ in probs])
    lda = (ctypes.c_int64 * n)(*[a.stride(0) for a, _, _, _ in probs])
    ldc = (ctypes.c_int64 * n)(*[c.stride(0) for _, _, c, _ in probs])
    N = (ctypes.c_int * n)(*[b.N for _, b, _, _ in probs])
    K = (ctypes.c_int * n)(*[b.K for _, b, _, _ in probs])
    epi = (ctypes.c_int * n)(*[e for _, _, _, e in probs])
    return n, A, B, C, lda, ldc, N, K, epi


def _problems(dev, M, shapes, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    probs = []
    for N, K, epi in shapes:
        A = torch.randn(M, K, generator=g, device=dev).bfloat16()
        B = (torch.randn(N, K, generator=g, device=dev) / K ** 0.5).bfloat16()
        probs.append((A, PackedWeight(B), torch.full((M, N), 3.0, device=dev).bfloat16(), epi))
    return probs


def _with_workspace(M, probs, st):
    n, A, B, C, lda, ldc, N, K, epi = _arrays(M, probs)
    need = _lib.load().rwkv7_gemm_decode_workspace(M, n, N, K)
    ws = torch.empty(max(need, 1), dtype=torch.float32, device=probs[0][0].device)
    _lib.call("rwkv7_gemm_decode", M, n, A, B, C, lda, ldc, N, K, epi, P(ws.data_ptr()), ws.numel(), st)
    return need


def _no_alloc(M, probs, st):
    n, A, B, C, lda, ldc, N, K, epi = _arrays(M, probs)
    _lib.call("rwkv7_gemm_decode_noalloc", M, n, A, B, C, lda, ldc, N, K, epi, st)


def test_noalloc_equals_workspace_entry_point(gpu_device):
    dev = gpu_device
    # call 1: the 1.5B decode step's FFN value (2048 x 8192) at 32 rows with a
    # sigmoid LoRA down (256 x 2048), both split K; call 2: a smaller set (16 rows,
    # a 7.2B-like output projection and a tanh LoRA down)
    calls = [(32, [(2048, 8192, 0), (256, 2048, 3)], 11),
             (16, [(4096, 4096, 0), (128, 4096, 2)], 12)]
    for i, (M, shapes, seed) in enumerate(calls):
        print(f"[case] no-alloc call {i + 1}: M={M}, shapes {shapes}", flush=True)
        ref = _problems(dev, M, shapes, seed)
        got = [(a, b, c.clone(), e) for a, b, c, e in ref]
        st = _lib.stream_of(ref[0][0])
        need = _with_workspace(M, ref, st)
        assert 0 < need <= SCRATCH_FLOATS   # the sets exercise the scratch
        _no_alloc(M, got, st)
        torch.cuda.synchronize()
        for (_, _, c_ref, _), (_, _, c_got, _), shp in zip(ref, got, shapes):
            assert torch.equal(c_ref, c_got), f"call {i + 1}, shape {shp}"
            assert bool(torch.isfinite(c_got.float()).all())
