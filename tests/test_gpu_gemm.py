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


@pytest.mark.parametrize("M", [1, 20, 32, 33, 48, 64, 80, 100, 128, 160, 200, 256])
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



@pytest.mark.parametrize("M", [1, 33, 100, 256])
@pytest.mark.parametrize("seq", [False, True])
def test_partials_feed_row_kernels(gpu_device, M, seq):
    """rwkv7_gemm_decode_partials at the FFN value shape: the planes summed in
    order are the product (to the GEMM tolerance, against the grouped GEMM's own
    result, which may split K differently), and the next row kernels (shift_mix,
    final_norm with add_parts) summing the planes themselves give, bit for bit,
    what they give reading that in-order sum rounded to bf16 - the value a
    reduction launch would write.  seq: the rows form one sequence, so the token
    shift also reads the previous row's sum; else every row is its own sequence
    (decode)."""
    print(f"[case] gemm partials M={M} seq={seq}", flush=True)
    g = torch.Generator(device=gpu_device).manual_seed(100 + M)
    C, K = 2048, 8192
    A = torch.randn(M, K, generator=g, device=gpu_device).bfloat16()
    Bw = (torch.randn(C, K, generator=g, device=gpu_device) / K ** 0.5).bfloat16()
    pw = PackedWeight(Bw)
    st = _lib.stream_of(A)
    direct = torch.empty(M, C, device=gpu_device).bfloat16()
    RWKV7Model._gemm_group(M, [(A, pw, direct, 0)], st)
    ws, parts = RWKV7Model._gemm_partials(M, A, pw, st)
    assert parts == _lib.load().rwkv7_gemm_decode_partial_count(M, C, K) >= 1
    planes = ws[:parts * M * C].view(parts, M, C)
    tot = planes[0].clone()
    for q in range(1, parts):
        tot += planes[q]
    out = tot.bfloat16()
    r = ref(A, Bw, 0)
    assert close(out, r) and close(direct, r)

    code = _lib.dtype_code(torch.bfloat16)
    P = _lib.ptr
    x_in = torch.randn(M, C, generator=g, device=gpu_device)
    ln_w = torch.rand(C, generator=g, device=gpu_device) + 0.5
    ln_b = torch.randn(C, generator=g, device=gpu_device) * 0.1
    mix = torch.rand(7, C, generator=g, device=gpu_device)
    row_slot = torch.arange(M, dtype=torch.int32, device=gpu_device)
    if seq:
        row_slot = torch.zeros(M, dtype=torch.int32, device=gpu_device)
        row_last = torch.full((M,), -1, dtype=torch.int32, device=gpu_device)
        row_last[0] = M - 1
    else:
        row_last = torch.arange(M, dtype=torch.int32, device=gpu_device)
    pool0 = torch.randn(M, C, generator=g, device=gpu_device)
    res = []
    for add, n_parts, stride in [(out, 0, 0), (ws, parts, M * C)]:
        x_out = torch.empty(M, C, device=gpu_device)
        pool = pool0.clone()
        mixed = torch.empty(7, M, C, device=gpu_device).bfloat16()
        _lib.call("rwkv7_shift_mix", code, M, C, P(x_in), P(add), n_parts, stride, None, None, 0, None, None,
                  P(x_out), P(ln_w), P(ln_b), P(pool), M, P(row_slot), P(row_last), 7, P(mix), P(mixed), st)
        rows = torch.arange(M - 1, -1, -1, dtype=torch.int32, device=gpu_device)
        y = torch.empty(M, C, device=gpu_device).bfloat16()
        _lib.call("rwkv7_final_norm", code, M, C, P(x_in), P(add), n_parts, stride, P(rows), P(ln_w), P(ln_b),
                  P(y), st)
        res.append((x_out, pool, mixed, y))
    torch.cuda.synchronize()
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_reduce_ragged_columns(gpu_device):
    """Split-K reduction of a problem whose N is not a multiple of 4 (element-wise
    path of gemm_reduce_kernel)."""
    g = torch.Generator(device=gpu_device).manual_seed(11)
    M, N, K = 3, 97, 4096
    A = torch.randn(M, K, generator=g, device=gpu_device).bfloat16()
    B = (torch.randn(N, K, generator=g, device=gpu_device) / K ** 0.5).bfloat16()
    C = torch.empty(M, N, device=gpu_device).bfloat16()
    N_, K_ = (ctypes.c_int * 1)(N), (ctypes.c_int * 1)(K)
    assert _lib.load().rwkv7_gemm_decode_workspace(M, 1, N_, K_) > 0  # the plan splits K
    RWKV7Model._gemm_group(M, [(A, PackedWeight(B), C, 0)], _lib.stream_of(C))
    torch.cuda.synchronize()
    assert close(C, ref(A, B, 0))

