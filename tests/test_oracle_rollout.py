"""Pins the CPU rollout oracle (oracle/rollout.py) against an independent
statement of the same sequences: each prompt decoded on its own, greedily, by
``oracle.model.greedy_generate`` (one batched prefill, then one token per step,
no forking, no live-list bookkeeping), then cut where the reference's stop rule
ends the path.  A mistake in the oracle's fork, lockstep batching, state
write-back or stop rule changes some path's tokens.  Also checks the
``SamplingParams`` validation of ``rwkvtune/sampling_params.py:45-60``."""

import pytest
import torch

from oracle import model as om
from oracle import rollout as orl
from rwkvtune_amd.model import RWKV7Config, build_model
from rwkvtune_amd.sampling_params import SamplingParams

V = 300


@pytest.fixture(scope="module")
def sd():
    cfg = RWKV7Config(n_layer=2, n_embd=256, vocab_size=V, dim_att_lora=32, dim_gate_lora=64, dim_mv_lora=32)
    m = build_model(cfg, dtype=torch.float32, device="cpu", seed=31)
    return om.cast_state_dict(m.state_dict(), torch.float32)


def _prompts(seed, lens):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, V - 3, (n,), generator=g).tolist() for n in lens]


def _isolated(sd, p, n_new):
    toks, _ = om.greedy_generate(sd, torch.tensor([p]), n_new, max_valid_id=V - 4)
    return toks[0].tolist()


def _cut_grpo(seq, eos, cap):
    """GRPO stop rule (grpo_batch_generator.py:283-285, 466-471): the first token
    never ends a path; a later EOS or reaching the cap does."""
    n = max(cap, 2)
    for i in range(1, len(seq)):
        if seq[i] == eos:
            n = min(n, i + 1)
            break
    return seq[:n]


def _cut_scheduler(seq, eos, cap):
    """SchedulerCore stop rule (scheduler_core.py:90-108): any EOS, the first
    token included, or max_new_tokens tokens."""
    for i, t in enumerate(seq[:cap]):
        if t == eos:
            return seq[:i + 1]
    return seq[:cap]


def test_grpo_rollout_equals_isolated_greedy(sd):
    ps = _prompts(1, [5, 9, 3])
    ps = [ps[0], ps[1], ps[0], ps[2]]            # a duplicate prompt
    iso = {tuple(p): _isolated(sd, p, 9) for p in ps}
    eos = iso[tuple(ps[1])][3]                    # ends prompt 1's paths after 4 tokens
    caps = [7, 1, 4, 9, 2, 6, 3, 5]               # G = 2 paths per prompt; cap 1 still gives 2 tokens
    toks, steps = orl.grpo_rollout(sd, ps, 9, 2, eos=eos, max_valid_id=V - 4, caps=caps)
    assert len(toks) == 8
    for q, t in enumerate(toks):
        want = _cut_grpo(iso[tuple(ps[q // 2])], eos, caps[q])
        assert t == want, (q, t, want)
    assert len(toks[3]) == 4 and toks[3][-1] == eos
    assert len(toks[1]) == 2
    # lockstep decode runs until the longest path ends
    assert steps == max(len(t) for t in toks) - 1


def test_grpo_rollout_paths_of_one_prompt_agree(sd):
    ps = _prompts(2, [6])
    toks, _ = orl.grpo_rollout(sd, ps, 6, 3, max_valid_id=V - 4)
    assert toks[0] == toks[1] == toks[2] == _isolated(sd, ps[0], 6)


def test_scheduler_rollout_equals_isolated_greedy(sd):
    ps = _prompts(3, [4, 7, 2])
    iso = [_isolated(sd, p, 8) for p in ps]
    eos = iso[2][0]                               # prompt 2 ends on its first token
    toks = orl.scheduler_rollout(sd, ps, 8, eos=eos, max_valid_id=V - 4)
    for t, s in zip(toks, iso):
        assert t == _cut_scheduler(s, eos, 8)
    assert toks[2] == [eos]
    toks1 = orl.scheduler_rollout(sd, ps, 1, max_valid_id=V - 4)
    assert toks1 == [[s[0]] for s in iso]


def test_sampling_params_validation():
    SamplingParams()
    SamplingParams(temperature=0.0, top_p=0.0, top_k=0, max_tokens=1)
    for kw in ({"temperature": -0.1}, {"top_p": 1.01}, {"top_p": -0.01}, {"top_k": -1}, {"max_tokens": 0}):
        with pytest.raises(ValueError):
            SamplingParams(**kw)
    sp = SamplingParams(stop=None, stop_token_ids=None, logit_bias={"65530": -100})
    assert sp.stop == [] and sp.stop_token_ids == []
    d = sp.to_dict()
    assert set(d) == {"max_tokens", "temperature", "top_p", "top_k", "stop", "stop_token_ids",
                      "skip_special_tokens", "repetition_penalty", "logit_bias"}
    assert SamplingParams.from_dict({**d, "unknown": 1}) == sp
