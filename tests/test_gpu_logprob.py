"""GRPO log-prob recompute on the GPU against the restated reference
(oracle/logprob.py).

Tolerances: float32 logits within 1e-5 absolute (one float32 logsumexp of up
to 65536 terms in a different order); bf16 / fp16 logits within one ulp of the
output dtype at the result (the float32 logsumexp may round the other way when
cast to the dtype); the fp32 model within 1e-4 of the fp64 oracle model, the
bf16 model within 3e-2 of the rows' logp (its activations are rounded to bf16
at every GEMM boundary, as in the reference).
"""

import pytest
import torch

from oracle import logprob as olp
from oracle import model as om
from rwkvtune_amd import grpo_utils
from rwkvtune_amd.model import RWKV7Config, build_model

pytestmark = pytest.mark.gpu


def ulp(x: torch.Tensor, dtype) -> torch.Tensor:
    return torch.finfo(dtype).eps * x.float().abs().clamp_min(torch.finfo(dtype).tiny)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("V", [65536, 1000, 37])
def test_selective_log_softmax_kernel(gpu_device, dtype, V):
    print(f"[case] selective_log_softmax {dtype} V={V}", flush=True)
    g = torch.Generator().manual_seed(V)
    x = (torch.randn(3, 41, V, generator=g) * 3).to(dtype)
    x[0, 0, :V // 2] = -float("inf")            # a row with banned entries
    idx = torch.randint(V // 2, V, (3, 41), generator=g)
    exp = olp.selective_log_softmax(x, idx)
    got = grpo_utils.selective_log_softmax(x.to(gpu_device), idx.to(gpu_device)).cpu()
    assert got.dtype == dtype and got.shape == (3, 41)
    d = (got.float() - exp.float()).abs()
    if dtype == torch.float32:
        assert float(d.max()) <= 1e-5
    else:
        assert bool((d <= ulp(exp, dtype) + 1e-6).all()), float(d.max())


def test_selective_log_softmax_strided_rows(gpu_device):
    """Rows with a stride larger than V (a slice of wider logits) and an odd offset."""
    g = torch.Generator().manual_seed(5)
    big = torch.randn(20, 530, generator=g).bfloat16()
    x = big[:, 3:515]
    idx = torch.randint(0, 512, (20,), generator=g)
    exp = olp.selective_log_softmax(x.contiguous(), idx)
    got = grpo_utils.selective_log_softmax(big.to(gpu_device)[:, 3:515], idx.to(gpu_device)).cpu()
    assert bool(((got.float() - exp.float()).abs() <= ulp(exp, torch.bfloat16) + 1e-6).all())


def tiny(dtype, seed, L=2, C=256, V=300, ctx_len=1024):
    cfg = RWKV7Config(n_layer=L, n_embd=C, vocab_size=V, ctx_len=ctx_len, dim_att_lora=32, dim_gate_lora=64,
                      dim_mv_lora=32)
    return build_model(cfg, dtype=dtype, device="cuda", seed=seed)


@pytest.mark.parametrize("P,C,ctx", [(9, 7, 1024), (20, 12, 1024), (30, 7, 24)])
def test_per_token_logps_fp32(gpu_device, P, C, ctx):
    """No padding / padding to 16 / prompt cut plus truncation, against the fp64
    oracle recompute; batch_size and row_chunk splits agree to float32 rounding."""
    print(f"[case] per-token logps P={P} C={C} ctx={ctx}", flush=True)
    m = tiny(torch.float32, seed=21, ctx_len=ctx)
    sd = om.cast_state_dict(m.state_dict(), torch.float64)
    V = m.config.vocab_size
    g = torch.Generator().manual_seed(P * 100 + C)
    pr = torch.randint(0, V, (5, P), generator=g)
    co = torch.randint(0, V, (5, C), generator=g)
    exp = olp.per_token_logps(sd, pr, co, ctx_len=ctx)
    got = grpo_utils.compute_per_token_logps(m, pr, co).cpu()
    assert got.shape == (5, C) and got.dtype == torch.float32
    assert float((got.double() - exp).abs().max()) <= 1e-4
    # other splits change the library GEMMs' row counts (and so possibly their
    # summation order), not the result beyond float32 rounding
    got2 = grpo_utils.compute_per_token_logps(m, pr, co, batch_size=2, row_chunk=3).cpu()
    assert float((got - got2).abs().max()) <= 1e-5


def test_per_token_logps_bf16(gpu_device):
    print("[case] per-token logps bf16 model", flush=True)
    m = tiny(torch.bfloat16, seed=22)
    sd = om.cast_state_dict(m.state_dict(), torch.float64)
    V = m.config.vocab_size
    g = torch.Generator().manual_seed(7)
    pr = torch.randint(0, V, (4, 33), generator=g)
    co = torch.randint(0, V, (4, 19), generator=g)
    exp = olp.per_token_logps(sd, pr, co, ctx_len=1024)
    got = grpo_utils.compute_per_token_logps(m, pr, co).cpu()
    assert got.dtype == torch.bfloat16
    assert float((got.double() - exp).abs().max()) <= 3e-2 * float(exp.abs().max())
