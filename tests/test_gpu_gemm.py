"""Grouped decode GEMM (rwkv7_gemm_decode over weights packed by
rwkv7_gemm_pack) against torch float32 matmul of the same bf16 operands.

Tolerance: the kernel accumulates in float32 and rounds once to bf16, so every
element must be within one bf16 ulp (2^-8 relative) of the rounded float32
reference, plus 1e-3 of the row's largest magnitude for accumulation-order
differences near zero.
"""

import ctypes

import pytest
import torch

from rwkvtune_amd import _lib
from rwkvtune_amd.model import PackedWeight, RWKV7Model

pytestmark = pytest.mark.gpu


def ref(A, B, epi):
    c = A.float() @ B.float().T
    if epi == 1:
        c = torch.relu(c) ** 2
    elif epi == 2:
        c = torch.tanh(c)
    elif epi == 3:
        c = torch.sigmoid(c)
    return c


def close(c, r):
    ulp = torch.pow(2.0, torch.floor(torch.log2(r.abs().clamp_min(1e-30))) - 7)
    tol = ulp + 1e-3 * r.abs().amax(dim=1, keepdim=True)
    return bool(((c.float() - r).abs() <= tol).all())


@pytest.mark.parametrize("M", [1, 20, 32, 33, 64, 100, 200, 256])
def test_grouped_gemm(gpu_device, M):
    """Shapes of the decode step (r/k/v, LoRA downs with tanh / sigmoid, FFN
    key with relu^2, FFN value, head slice) plus K tails (K % 64 != 0) and an
    N that is not a multiple of the tile."""
    print(f"[case] grouped gemm M={M}", flush=True)
    g = torch.Generator(device=gpu_device).manual_seed(M)
    shapes = [(2048, 2048, 0), (96, 2048, 2), (2048, 96, 0), (256, 2048, 3), (2048, 256, 0),
              (200, 160, 1), (8192, 2048, 1), (2048, 8192, 0), (300, 8, 0), (4096, 2048, 0)]
    probs = []
    for N, K, epi in shapes:
        A = torch.randn(M, K, generator=g, device=gpu_device).bfloat16()
        B = (torch.randn(N, K, generator=g, device=gpu_device) / K ** 0.5).bfloat16()
        C = torch.full((M, N), 7.0, device=gpu_device).bfloat16()
        probs.append((A, B, C, epi))
    st = _lib.stream_of(probs[0][0])
    packed = [(A, PackedWeight(B), C, epi) for A, B, C, epi in probs]
    RWKV7Model._gemm_group(M, packed[:4], st)
    RWKV7Model._gemm_group(M, packed[4:8], st)
    for p in packed[8:]:
        RWKV7Model._gemm_group(M, [p], st)
    torch.cuda.synchronize()
    for (A, B, C, epi), shp in zip(probs, shapes):
        assert close(C, ref(A, B, epi)), f"shape {shp}"


def test_pack_layout(gpu_device):
    """The packed layout, element by element: tile (nt, kt) at (nt*KT + kt)*4096,
    row r of a tile holds B[64 nt + r][64 kt + 8 (p ^ s(r)) ..] at chunk p with
    s(r) = (r ^ (r >> 3)) & 7, zero padding past N and K."""
    g = torch.Generator(device=gpu_device).manual_seed(3)
    N, K = 100, 136
    B = torch.randn(N, K, generator=g, device=gpu_device).bfloat16()
    pw = PackedWeight(B)
    KT, NT = (K + 63) // 64, (N + 63) // 64
    assert pw.t.numel() == NT * 64 * KT * 64
    got = pw.t.view(NT, KT, 64, 8, 8).cpu()
    ref_full = torch.zeros(NT * 64, KT * 64, dtype=torch.bfloat16)
    ref_full[:N, :K] = B.cpu()
    for r in range(64):
        s = (r ^ (r >> 3)) & 7
        for p in range(8):
            c = p ^ s
            exp = ref_full.view(NT, 64, KT, 8, 8)[:, r, :, c, :]
            assert torch.equal(got[:, :, r, p, :], exp), (r, p)


def test_operand_checks(gpu_device):
    A = torch.zeros(4, 64, device=gpu_device).bfloat16()
    pw = PackedWeight(torch.zeros(32, 64, device=gpu_device).bfloat16())
    C = torch.zeros(4, 32, device=gpu_device).bfloat16()
    with pytest.raises(ValueError):
        RWKV7Model._gemm_group(5, [(A, pw, C, 0)], _lib.stream_of(A))
    with pytest.raises(ValueError):
        RWKV7Model._gemm_group(4, [(A.float(), pw, C, 0)], _lib.stream_of(A))


def test_strided_operands(gpu_device):
    """A as a view with a row stride larger than K (a slice of a wider buffer)."""
    g = torch.Generator(device=gpu_device).manual_seed(9)
    big = torch.randn(37, 3 * 512, generator=g, device=gpu_device).bfloat16()
    A = big[:, 512:1024]
    B = torch.randn(300, 512, generator=g, device=gpu_device).bfloat16()
    C = torch.empty(37, 300, device=gpu_device).bfloat16()
    RWKV7Model._gemm_group(37, [(A, PackedWeight(B), C, 0)], _lib.stream_of(C))
    torch.cuda.synchronize()
    assert close(C, ref(A, B, 0))

