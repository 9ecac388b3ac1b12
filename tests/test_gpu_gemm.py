"""Grouped decode GEMM (rwkv7_gemm_decode) against torch float32 matmul of the
same bf16 operands.

Tolerance: the kernel accumulates in float32 and rounds once to bf16, so every
element must be within one bf16 ulp (2^-8 relative) of the rounded float32
reference, plus 1e-3 of the row's largest magnitude for accumulation-order
differences near zero.
"""

import ctypes

import pytest
import torch

from rwkvtune_amd import _lib
from rwkvtune_amd.model import RWKV7Model

pytestmark = pytest.mark.gpu


def ref(A, B, act, epi):
    a = A.float()
    if act == 1:
        a = torch.tanh(a).bfloat16().float()
    elif act == 2:
        a = torch.sigmoid(a).bfloat16().float()
    c = a @ B.float().T
    if epi == 1:
        c = torch.relu(c) ** 2
    return c


def close(c, r):
    ulp = torch.pow(2.0, torch.floor(torch.log2(r.abs().clamp_min(1e-30))) - 7)
    tol = ulp + 1e-3 * r.abs().amax(dim=1, keepdim=True)
    return bool(((c.float() - r).abs() <= tol).all())


@pytest.mark.parametrize("M", [1, 20, 64, 256])
def test_grouped_gemm(gpu_device, M):
    print(f"[case] grouped gemm M={M}", flush=True)
    g = torch.Generator(device=gpu_device).manual_seed(M)
    shapes = [(2048, 2048, 0, 0), (96, 2048, 0, 0), (2048, 96, 1, 0), (256, 2048, 0, 0), (2048, 256, 2, 0),
              (200, 160, 0, 1), (8192, 2048, 0, 1)]
    probs = []
    for N, K, act, epi in shapes:
        A = torch.randn(M, K, generator=g, device=gpu_device).bfloat16()
        B = (torch.randn(N, K, generator=g, device=gpu_device) / K ** 0.5).bfloat16()
        C = torch.full((M, N), 7.0, device=gpu_device).bfloat16()
        probs.append((A, B, C, act, epi))
    st = _lib.stream_of(probs[0][0])
    RWKV7Model._gemm_group(M, probs[:4], st)
    RWKV7Model._gemm_group(M, probs[4:], st)
    torch.cuda.synchronize()
    for (A, B, C, act, epi), shp in zip(probs, shapes):
        assert close(C, ref(A, B, act, epi)), f"shape {shp}"


def test_strided_operands(gpu_device):
    """A as a view with a row stride larger than K (a slice of a wider buffer)."""
    g = torch.Generator(device=gpu_device).manual_seed(9)
    big = torch.randn(37, 3 * 512, generator=g, device=gpu_device).bfloat16()
    A = big[:, 512:1024]
    B = torch.randn(300, 512, generator=g, device=gpu_device).bfloat16()
    C = torch.empty(37, 300, device=gpu_device).bfloat16()
    RWKV7Model._gemm_group(37, [(A, B, C, 0, 0)], _lib.stream_of(C))
    torch.cuda.synchronize()
    assert close(C, ref(A, B, 0, 0))
