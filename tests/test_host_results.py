"""Host-side assembly of rollout results (no GPU): the per-sequence lists of
``RolloutResult`` and the padded ids / masks that ``GRPOBatchGenerator.generate``
returns, against a plain restatement of the reference's ``_collect_results``
(rwkvtune/inference/grpo_batch_generator.py:680-750): ids padded with 0 to the
longest sequence ([[0]] per sequence when nothing was generated), mask True on
the generated positions, completions decoded per sequence."""
from types import SimpleNamespace

import torch

from rwkvtune_amd.engine import RolloutResult
from rwkvtune_amd.grpo_batch_generator import GRPOBatchGenerator


def reference_collect(tokens, decode):
    max_len = max((len(t) for t in tokens), default=0)
    if max_len == 0:
        return [""] * len(tokens), torch.zeros((len(tokens), 1), dtype=torch.long), \
            torch.zeros((len(tokens), 1), dtype=torch.bool)
    completions = [decode(t) if t else "" for t in tokens]
    ids = torch.tensor([t + [0] * (max_len - len(t)) for t in tokens], dtype=torch.long)
    masks = torch.zeros_like(ids, dtype=torch.bool)
    for i, t in enumerate(tokens):
        masks[i, :len(t)] = True
    return completions, ids, masks


def make_result(ngen, maxlen, seed=0):
    g = torch.Generator().manual_seed(seed)
    n = len(ngen)
    tok = torch.randint(0, 65530, (n, maxlen), generator=g, dtype=torch.int32)
    logp = -torch.rand((n, maxlen), generator=g)
    step = torch.randint(0, 1000, (n, maxlen), generator=g, dtype=torch.int32)
    return RolloutResult(ngen, tok, logp, step, n_decode_steps=7), tok, logp, step


def test_lists_are_row_prefixes():
    ngen = [3, 0, 9, 1, 9]
    res, tok, logp, step = make_result(ngen, 9)
    for q, g in enumerate(ngen):
        assert res.tokens[q] == tok[q, :g].tolist()
        assert res.logps[q] == logp[q, :g].tolist()
        assert res.steps[q] == step[q, :g].tolist()
    assert res.tokens is res.tokens  # built once


def test_padded_ids_match_reference_collect():
    for seed, ngen in enumerate([[3, 0, 9, 1, 9], [1], [5, 5, 5], [0, 2, 0, 7]]):
        res, _, _, _ = make_result(ngen, 9, seed)
        _, ids_ref, mask_ref = reference_collect(res.tokens, str)
        ids, mask = res.padded_ids()
        assert ids.dtype == torch.long and mask.dtype == torch.bool
        assert torch.equal(ids, ids_ref) and torch.equal(mask, mask_ref)


def test_nothing_generated():
    res, _, _, _ = make_result([0, 0, 0], 4)
    ids, mask = res.padded_ids()
    assert ids.shape == (3, 1) and not ids.any() and not mask.any()
    empty = RolloutResult([], None, None, None, 0)
    assert empty.tokens == [] and empty.padded_ids()[0].shape == (0, 1)


class _Tok:
    """decode() fails on id 7 (KeyError), as a tokenizer can on an unknown id; the
    reference then joins idx2token pieces (grpo_batch_generator.py:697-706)."""
    idx2token = {7: b"<7>"}

    def decode(self, ids):
        if 7 in ids:
            raise KeyError(7)
        return ",".join(str(i) for i in ids)


def test_generator_collect_results():
    ngen = [4, 0, 6, 2]
    res, tok, _, _ = make_result(ngen, 6, seed=3)
    tok[2, 1] = 7  # exercises the fallback on row 2
    stub = SimpleNamespace(tokenizer=_Tok(), device=torch.device("cpu"))
    out = GRPOBatchGenerator._collect_results(stub, res)

    def ref_decode(ids):
        try:
            return _Tok().decode(ids)
        except KeyError:
            return b"".join(_Tok.idx2token.get(t, b"?") for t in ids).decode("utf-8", errors="replace")

    comps, ids_ref, mask_ref = reference_collect(res.tokens, ref_decode)
    assert out["completions"] == comps
    assert torch.equal(out["completion_ids"], ids_ref) and torch.equal(out["masks"], mask_ref)
    stub.tokenizer = None
    assert GRPOBatchGenerator._collect_results(stub, res)["completions"] == [""] * len(ngen)
