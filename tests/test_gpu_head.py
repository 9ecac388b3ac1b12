"""LM head GEMM (rwkv7_head_logits over a weight packed by rwkv7_head_pack)
against torch float32 matmul of the same bf16 operands, and the model's decode
logits on it.

Tolerance: the kernel accumulates in float32 and rounds once to bf16, so every
element must be within one bf16 ulp (2^-8 relative) of the rounded float32
reference, plus 1e-3 of the row's largest magnitude for accumulation-order
differences near zero (the tolerance of the decode GEMM's tests).
"""

import ctypes

import pytest
import torch

from rwkvtune_amd import _lib
from rwkvtune_amd.model import HeadPack, build_model, config_from_preset

pytestmark = pytest.mark.gpu


def close(c, r):
    ulp = torch.pow(2.0, torch.floor(torch.log2(r.abs().clamp_min(1e-30))) - 7)
    tol = ulp + 1e-3 * r.abs().amax(dim=1, keepdim=True)
    return bool(((c.float() - r).abs() <= tol).all())


def test_head_pack_layout(gpu_device):
    """Piece (g, kt) at element (g * K/32 + kt) * 2048 holds rows 64 g .. +63,
    columns 32 kt .. +31 row-major; rows past V are zero."""
    g = torch.Generator(device=gpu_device).manual_seed(5)
    V, K = 300, 128
    W = torch.randn(V, K, generator=g, device=gpu_device).bfloat16()
    Wp = torch.empty(_lib.load().rwkv7_head_packed_elems(V, K), dtype=torch.bfloat16, device=gpu_device)
    _lib.call("rwkv7_head_pack", _lib.ptr(W), W.stride(0), V, K, _lib.ptr(Wp), _lib.stream_of(W))
    torch.cuda.synchronize()
    G = (V + 63) // 64
    full = torch.zeros(G * 64, K, dtype=torch.bfloat16, device=gpu_device)
    full[:V] = W
    ref = full.view(G, 64, K // 32, 32).permute(0, 2, 1, 3).reshape(-1)
    assert Wp.numel() == G * 64 * K
    assert torch.equal(Wp, ref)


def head_case(dev, M, V, K, seed, lda_pad=0, ldc_pad=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    A = torch.randn(M, K + lda_pad, generator=g, device=dev).bfloat16()[:, :K]
    W = (torch.randn(V, K, generator=g, device=dev) / K ** 0.5).bfloat16()
    hp = HeadPack(W)
    out = torch.full((M, V + ldc_pad), 7.0, device=dev).bfloat16()
    _lib.call("rwkv7_head_logits", M, V, K, _lib.ptr(A), A.stride(0), _lib.ptr(hp.t), _lib.ptr(out),
              out.stride(0), _lib.stream_of(A))
    torch.cuda.synchronize()
    ref = A.float() @ W.float().T
    return out, ref, A, W


@pytest.mark.parametrize("M", [1, 7, 32, 63, 64, 65, 100, 128, 130, 256])
def test_head_logits_cfg4_shape(gpu_device, M):
    """The 1.5B head (65,536 x 2,048): both row tiles (64 and 128 rows), row
    counts off the tile, and row counts above 128 (several row tiles)."""
    print(f"[case] head logits M={M} V=65536 K=2048", flush=True)
    out, ref, A, W = head_case(gpu_device, M, 65536, 2048, seed=M)
    assert close(out, ref)


@pytest.mark.parametrize("M,V,K,lda_pad,ldc_pad", [(128, 65536, 4096, 0, 0), (32, 65536, 4096, 64, 0),
                                                   (5, 512, 256, 8, 8), (70, 1024, 320, 0, 24),
                                                   (64, 256, 1024, 0, 0)])
def test_head_logits_shapes(gpu_device, M, V, K, lda_pad, ldc_pad):
    """The 7.2B head (K = 4,096), the smallest K (256) and V (256), K not a power
    of two, strided activations and logits (padding columns untouched)."""
    print(f"[case] head logits M={M} V={V} K={K} lda+{lda_pad} ldc+{ldc_pad}", flush=True)
    out, ref, A, W = head_case(gpu_device, M, V, K, seed=V + K + M, lda_pad=lda_pad, ldc_pad=ldc_pad)
    assert close(out[:, :V], ref)
    if ldc_pad:
        assert bool((out[:, V:].float() == 7.0).all())


def test_head_logits_rejects_bad_shapes(gpu_device):
    A = torch.zeros(4, 256, dtype=torch.bfloat16, device=gpu_device)
    Wp = torch.zeros(_lib.load().rwkv7_head_packed_elems(512, 256), dtype=torch.bfloat16, device=gpu_device)
    out = torch.zeros(4, 512, dtype=torch.bfloat16, device=gpu_device)
    lib = _lib.load()
    st = _lib.stream_of(A)
    P = _lib.ptr
    assert lib.rwkv7_head_logits(4, 500, 256, P(A), 256, P(Wp), P(out), 512, st) != 0  # V % 256
    assert lib.rwkv7_head_logits(4, 512, 192, P(A), 256, P(Wp), P(out), 512, st) != 0  # K < 256
    assert lib.rwkv7_head_logits(4, 512, 256, P(A), 100, P(Wp), P(out), 512, st) != 0  # lda < K
    assert lib.rwkv7_head_logits(4, 512, 256, P(A), 256, P(Wp), P(out), 256, st) != 0  # ldc < V
    misaligned = ctypes.c_void_p(A.data_ptr() + 2)
    assert lib.rwkv7_head_logits(4, 512, 256, misaligned, 256, P(Wp), P(out), 512, st) != 0  # alignment
    assert lib.rwkv7_head_logits(0, 512, 256, P(A), 256, P(Wp), P(out), 512, st) == 0  # no rows: nothing to do
    assert lib.rwkv7_head_packed_elems(512, 100) == -1


def test_model_decode_logits_on_head_kernel(gpu_device):
    """A bf16 model with a 65,536-token vocabulary decodes its logits on the head
    kernel (rows <= 128) and equals the library GEMM's logits to the tolerance;
    with the kernel switched off the model takes the library GEMM.  An in-place
    update of the head weight is picked up by the next forward (repack)."""
    cfg = config_from_preset("rwkv7-1.5b", n_layer=1, vocab_size=65536)
    m = build_model(cfg, dtype=torch.bfloat16, device="cuda", seed=9)
    tok = torch.randint(0, 65536, (48, 1), generator=torch.Generator().manual_seed(10)).to(gpu_device)
    st = m.init_state(48)
    logits, _ = m.forward_with_state(tok, st)
    assert m._head_pack is not None
    m.use_head_kernel = False
    ref_logits, _ = m.forward_with_state(tok, m.init_state(48))
    m.use_head_kernel = True
    assert close(logits.reshape(48, -1), ref_logits.reshape(48, -1).float())
    with torch.no_grad():
        m.head.weight.mul_(0.5)
    logits2, _ = m.forward_with_state(tok, m.init_state(48))
    m.use_head_kernel = False
    ref2, _ = m.forward_with_state(tok, m.init_state(48))
    assert close(logits2.reshape(48, -1), ref2.reshape(48, -1).float())
    assert not torch.equal(logits2, logits)
