"""CPU checks of the C ABI: the library loads, exports exactly what the header
declares, and rejects bad arguments on the host (no kernel is launched)."""

import ctypes
import os
import re
import subprocess

import pytest

from rwkvtune_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rwkv7_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rwkv7\w*)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("librwkv7_hip.so is not built (run python -m rwkvtune_amd.build)")
    return _lib.load()


def test_header_matches_exports(lib):
    decl = declared_functions()
    assert decl, "no functions parsed from the header"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = sorted(set(re.findall(r"\sT\s(rwkv7\w*)$", out, flags=re.M)))
    assert exported == decl
    assert sorted(_lib.SIGNATURES) == decl
    for name in decl:
        assert getattr(lib, name) is not None


def test_abi_version(lib):
    assert lib.rwkv7_abi_version() == 2


def _null6():
    return [None] * 6


def test_host_side_errors(lib):
    P = ctypes.c_void_p
    fake = P(16)  # never dereferenced: every call below fails before any launch
    # bad dtype
    rc = lib.rwkv7s_forward(7, 1, 1, 64, 1, fake, *[fake] * 6, fake, None)
    assert rc == 1 and b"dtype" in lib.rwkv7_last_error()
    # C != H*64 (a host assert in the reference kernel launcher)
    rc = lib.rwkv7s_forward(2, 1, 1, 96, 1, fake, *[fake] * 6, fake, None)
    assert rc == 1 and b"H*64" in lib.rwkv7_last_error()
    # null pointer
    rc = lib.rwkv7s_forward(2, 1, 1, 64, 1, None, *[fake] * 6, fake, None)
    assert rc == 1 and b"null" in lib.rwkv7_last_error()
    # empty problems succeed without touching the GPU
    assert lib.rwkv7s_forward(2, 0, 5, 64, 1, None, *_null6(), None, None) == 0
    assert lib.rwkv7_last_error() == b""
    assert lib.rwkv7_wkv_decode(2, 0, 1, None, 0, None, *_null6(), None, None) == 0
    # identity slots need a pool at least as large as the batch
    rc = lib.rwkv7_wkv_decode(2, 4, 1, fake, 2, None, *[fake] * 6, fake, None)
    assert rc == 1 and b"pool_slots" in lib.rwkv7_last_error()
    # prefill: chunk length outside {0,1,16,32,64}; missing cu_seqlens
    rc = lib.rwkv7_wkv_prefill(2, 1, 1, 4, fake, None, fake, 1, *[fake] * 6, fake, 48, None)
    assert rc == 1 and b"chunk_len" in lib.rwkv7_last_error()
    rc = lib.rwkv7_wkv_prefill(2, 1, 1, 4, None, None, fake, 1, *[fake] * 6, fake, 0, None)
    assert rc == 1 and b"cu_seqlens" in lib.rwkv7_last_error()
    # inputs must be aligned to 4 elements (8 bytes for bf16, 16 for fp32), the state to 16 bytes
    odd = P(16 + 2)
    rc = lib.rwkv7_wkv_prefill(2, 1, 1, 4, fake, None, fake, 1, odd, *[fake] * 5, fake, 0, None)
    assert rc == 1 and b"aligned" in lib.rwkv7_last_error()
    rc = lib.rwkv7_wkv_decode(0, 1, 1, fake, 1, None, *[fake] * 5, P(16 + 8), fake, None)
    assert rc == 1 and b"aligned" in lib.rwkv7_last_error()
    rc = lib.rwkv7s_forward(2, 1, 2, 64, 1, P(16 + 8), *[fake] * 6, fake, None)
    assert rc == 1 and b"aligned" in lib.rwkv7_last_error()


def test_python_wrapper_raises_library_message(lib):
    with pytest.raises(ValueError, match="bad dtype"):
        _lib.call("rwkv7s_forward", 9, 1, 1, 64, 1, ctypes.c_void_p(16),
                  *[ctypes.c_void_p(16)] * 7, None)


def test_gemm_host_side_errors(lib):
    P = ctypes.c_void_p
    fake = P(16)
    # packed size: 64 x 64 tiles, zero padding; invalid sizes give -1 and a message
    assert lib.rwkv7_gemm_packed_elems(100, 136) == 128 * 192
    assert lib.rwkv7_gemm_packed_elems(64, 12) == -1 and b"K % 8" in lib.rwkv7_last_error()
    # pack: ldb below K, misaligned output
    assert lib.rwkv7_gemm_pack(fake, 8, 16, 64, fake, None) == 1 and b"ldb" in lib.rwkv7_last_error()
    assert lib.rwkv7_gemm_pack(fake, 64, 16, 64, P(16 + 2), None) == 1
    # grouped GEMM: problem count, K % 8, lda below K, epilogue code
    one = (ctypes.c_int * 1)
    arr = (P * 1)
    i64 = (ctypes.c_int64 * 1)
    args = lambda N, K, lda, epi: (4, 1, arr(fake), arr(fake), arr(fake), i64(lda), i64(N), one(N), one(K),
                                   one(epi), None, 0, None)
    assert lib.rwkv7_gemm_decode(4, 0, *args(64, 64, 64, 0)[2:]) == 1
    assert lib.rwkv7_gemm_decode(*args(64, 60, 64, 0)) == 1 and b"K % 8" in lib.rwkv7_last_error()
    assert lib.rwkv7_gemm_decode(*args(64, 64, 32, 0)) == 1 and b"lda" in lib.rwkv7_last_error()
    assert lib.rwkv7_gemm_decode(*args(64, 64, 64, 5)) == 1 and b"epi" in lib.rwkv7_last_error()
    assert lib.rwkv7_gemm_decode_workspace(256, 1, one(2048), one(60)) == -1


def test_gemm_scratch_bound(lib):
    """rwkv7_gemm_decode_noalloc keeps split-K partials in a static scratch of
    RWKV7_GEMM_SCRATCH_FLOATS floats.  The split plan (a host computation) splits
    K only at M <= 32 rows, to about 256 blocks of at most 32 x 32 outputs, so no
    problem set needs more than 510 * 32 * 32 floats: swept here over every
    column count of one to eight problems on a 32-column grid, row counts 1 .. 64
    and deep K, and no plan above 32 rows splits at all."""
    scratch = 1 << 21   # RWKV7_GEMM_SCRATCH_FLOATS in include/rwkv7_hip.h
    bound = 510 * 32 * 32
    assert bound <= scratch
    worst = 0
    arr = lambda xs: (ctypes.c_int * len(xs))(*xs)
    for M in list(range(1, 65)) + [65, 96, 128, 200, 256, 1024]:
        for n in range(32, 16416, 32):
            for count in (1, 3, 8):
                need = lib.rwkv7_gemm_decode_workspace(M, count, arr([n] * count), arr([16384] * count))
                assert need >= 0
                worst = max(worst, need)
                if M > 32:
                    assert need == 0, (M, n, count)
    assert 0 < worst <= bound


def test_partials_host_side_errors(lib):
    P = ctypes.c_void_p
    fake = P(16)
    parts = ctypes.c_int32(0)
    pp = P(ctypes.addressof(parts))
    assert lib.rwkv7_gemm_decode_partial_count(4, 32, 12) == -1 and b"K % 8" in lib.rwkv7_last_error()
    n = lib.rwkv7_gemm_decode_partial_count(256, 2048, 8192)
    assert 1 <= n <= 8
    # workspace too small for n planes of 256 x 2048 floats; the count is reported anyway
    assert lib.rwkv7_gemm_decode_partials(256, fake, fake, 8192, 2048, 8192, fake, 10, pp, None) == 1
    assert parts.value == n and b"workspace" in lib.rwkv7_last_error()
    assert lib.rwkv7_gemm_decode_partials(256, fake, fake, 8192, 2048, 8192, fake, 1 << 30, None, None) == 1
    # row kernels: partial planes need x_in (not tokens), alignment and a stride of M * C floats
    row = (2, 4, 8, fake)  # dtype bf16, M, C, x_in
    rest = (None, None, 0, None, None, fake, fake, fake, fake, 4, fake, fake, 7, fake, fake, None)
    assert lib.rwkv7_shift_mix(*row, fake, 2, 8, *rest) == 1 and b"partial" in lib.rwkv7_last_error()
    assert lib.rwkv7_shift_mix(*row, P(18), 1, 0, *rest) == 1  # misaligned planes
    assert lib.rwkv7_shift_mix(*row, fake, 65, 32, *rest) == 1  # too many planes
    assert lib.rwkv7_final_norm(2, 4, 8, fake, fake, 2, 4, None, fake, fake, fake, None) == 1


def test_train_host_side_errors(lib):
    P = ctypes.c_void_p
    fake = P(16)
    assert lib.rwkv7_wkv_train_ckpt_floats(2, 33, 3) == 2 * 3 * 3 * 64 * 64
    assert lib.rwkv7_wkv_train_ckpt_floats(2, 33, 0) == -1
    ins = [fake] * 7  # r, w, k, v, a, b, y
    assert lib.rwkv7_wkv_train_forward(7, 1, 16, 1, *ins, None, None, fake, fake, None) == 1  # dtype
    assert lib.rwkv7_wkv_train_forward(2, 1, 16, 1, *ins, None, None, None, fake, None) == 1  # no ckpt
    assert lib.rwkv7_wkv_train_forward(2, 1, 16, 1, *ins, P(20), None, fake, fake, None) == 1  # misaligned s0
    assert b"aligned" in lib.rwkv7_last_error()
    assert lib.rwkv7_wkv_train_forward(2, 0, 16, 1, *ins, None, None, None, None, None) == 0  # empty batch
    grads = [fake] * 6
    assert lib.rwkv7_wkv_train_backward(2, 1, 16, 1, *[fake] * 7, fake, fake, None, *grads[:5], None, None,
                                        None) == 1  # null db


def test_training_operator_needs_gpu_tensors():
    import torch
    from rwkvtune_amd import operators as ops
    op = ops.load_wkv_operator(device="cuda", for_inference=False)
    assert op is ops.load_cuda_operator_train()
    x = torch.zeros(1, 16, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        op(x, x, x, x, x, x)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.rwkv7_wkv_infctx(*(x.view(1, 16, 1, 64),) * 6)
