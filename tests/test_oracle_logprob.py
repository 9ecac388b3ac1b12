"""Pins of the restated GRPO log-prob recompute (oracle/logprob.py) on the CPU."""

import math

import torch

from oracle import logprob as olp


def test_selective_log_softmax_identities():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 7, 300, generator=g, dtype=torch.float64) * 4
    V = x.shape[-1]
    # all indices: probabilities sum to 1
    idx = torch.arange(V).expand(5, 7, V)
    lp = torch.stack([olp.selective_log_softmax(x, idx[..., i]) for i in range(V)], -1)
    assert torch.allclose(lp.exp().sum(-1), torch.ones(5, 7, dtype=torch.float64), atol=1e-12)
    # agreement with log_softmax + gather, shift invariance
    i = torch.randint(0, V, (5, 7), generator=g)
    ref = torch.log_softmax(x, -1).gather(-1, i[..., None])[..., 0]
    assert torch.allclose(olp.selective_log_softmax(x, i), ref, atol=1e-12)
    assert torch.allclose(olp.selective_log_softmax(x + 123.0, i), ref, atol=1e-10)
    # closed forms: uniform row, one dominant logit
    u = torch.zeros(3, 1000, dtype=torch.float64)
    assert torch.allclose(olp.selective_log_softmax(u, torch.tensor([0, 5, 999])),
                          torch.full((3,), -math.log(1000.0), dtype=torch.float64))
    d = torch.zeros(1, 50, dtype=torch.float64)
    d[0, 7] = 60.0
    assert abs(float(olp.selective_log_softmax(d, torch.tensor([7]))[0])) < 1e-20


def test_selective_log_softmax_bf16_rule():
    """bf16 rows: float32 logsumexp, rounded to bf16, subtracted in bf16."""
    x = torch.tensor([[1.0, 2.0, 3.0, 4.0], [0.5, 0.5, 0.5, 10.0]]).bfloat16()
    i = torch.tensor([2, 3])
    got = olp.selective_log_softmax(x, i)
    assert got.dtype == torch.bfloat16
    lse = torch.logsumexp(x.float(), -1).bfloat16()
    exp = (x.float().gather(-1, i[:, None])[:, 0] - lse.float()).bfloat16()
    assert torch.equal(got, exp)
    # hand check of row 0: lse = 4 + log(1 + e^-1 + e^-2 + e^-3) = 4.4402 -> bf16 4.4375
    assert float(lse[0]) == 4.4375
    assert float(got[0]) == float(torch.tensor(3.0 - 4.4375).bfloat16())


def test_build_inputs_shapes():
    P, C = 10, 7
    pr = torch.arange(1, P + 1)[None].repeat(2, 1)
    co = torch.arange(100, 100 + C)[None].repeat(2, 1)
    # no cut: 10 + 6 = 16 tokens, already a multiple of 16
    ids, keep, c = olp.build_inputs(pr, co, ctx_len=1024)
    assert ids.shape == (2, 16) and keep == 7 and c == 7
    assert ids[0, :10].tolist() == list(range(1, 11)) and ids[0, 10:].tolist() == list(range(100, 106))
    # padding: 10 + 4 = 14 -> 16, keep = C + 2
    ids, keep, c = olp.build_inputs(pr, co[:, :5], ctx_len=1024)
    assert ids.shape == (2, 16) and keep == 7 and ids[0, 14:].tolist() == [0, 0]
    # prompt cut to ctx_len - (C - 1) = 12 - 6 = 6 leading tokens, 12 -> pad would make 16 > 12:
    # truncation to 12 // 16 * 16 = 0 ... use ctx_len 20: prompt cut to 14, 14 + 6 = 20 -> 32 > 20 -> 16
    big = torch.arange(1, 31)[None]
    ids, keep, c = olp.build_inputs(big, co[:1], ctx_len=20)
    assert ids.shape == (1, 16) and keep == 7
    assert ids[0].tolist() == list(range(1, 15)) + [100, 101]


def test_per_token_logps_matches_full_forward():
    """The recompute equals log_softmax of a plain full forward at the positions
    that predict each completion token (fp64 oracle model)."""
    from oracle import model as om
    from tests.test_oracle_model import tiny_sd
    sd = tiny_sd(seed=3)
    V = sd["emb.weight"].shape[0]
    g = torch.Generator().manual_seed(4)
    pr = torch.randint(0, V, (2, 9), generator=g)
    co = torch.randint(0, V, (2, 5), generator=g)
    got = olp.per_token_logps(sd, pr, co, ctx_len=1024)
    full = torch.cat([pr, co], 1)
    logits, _ = om.forward_with_state(sd, full, None)
    ref = torch.log_softmax(logits, -1)[:, 8:13].gather(-1, co[..., None])[..., 0]
    assert torch.allclose(got, ref, atol=1e-10)
