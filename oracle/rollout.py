"""CPU restatement of the reference rollout loops (test infrastructure and the
timed CPU baseline; see ``oracle/__init__``).

``grpo_rollout`` follows ``rwkvtune/inference/grpo_batch_generator.py:115-610``:
dedupe prompts (``:152-161``), prefill each distinct prompt (the reference groups
by exact length; per-prompt prefill gives the same states), fork the state to the
G paths (``:233-260``), first token with the single-sample rules from the prompt's
last logits (``:262-285``), then lockstep decode of the unfinished paths, one
``forward_with_state`` per step (``:458-610``), ending a path on EOS or at its
token cap; the first token never ends a path (``:283-285`` vs ``:466-471``).

``scheduler_rollout`` follows ``rwkvtune/inference/scheduler_core.py`` semantics
per sequence: first token from the prefill logits, every token with the
single-sample rules, finished on EOS or ``max_new_tokens`` tokens (``:90-108``),
the first token included.

Greedy decoding (temperature 0) makes both deterministic, which is what the
parity tests compare.  Sampled decoding uses ``torch.multinomial`` on the rule's
distribution (``oracle.sampler.distribution``); it is only used for timing.

Pinning (tests/test_oracle_rollout.py): every greedy path equals its prompt
decoded alone by ``oracle.model.greedy_generate`` (no fork, no lockstep batch),
cut by the stop rule - with duplicate prompts, per-path caps (cap 1 giving two
tokens in GRPO), an EOS that ends some paths mid-way and one that ends a
scheduler sequence on its first token; the lockstep loop runs exactly until the
longest path ends.  A wrong cap comparison, a lost state write-back, a fork
from the wrong prompt or a dropped EOS check each fails one of them.
"""

from __future__ import annotations

import torch

from . import model as om
from . import sampler as osm


def _pick(logits_row, temperature, top_p, top_k, max_valid_id, rule, gen=None):
    if temperature == 0 or temperature < 1e-6:
        return osm.greedy(logits_row, max_valid_id)[0]
    d = osm.distribution(logits_row, temperature, top_p, top_k, None, max_valid_id, rule)
    return int(torch.multinomial(d, 1, generator=gen))


def _batch_pick(logits, temperature, top_p, top_k, max_valid_id, rule, gen=None):
    return [_pick(logits[i], temperature, top_p, top_k, max_valid_id, rule, gen) for i in range(logits.shape[0])]


def _fork(states, idx):
    return [{k: v[idx].clone() for k, v in layer.items()} for layer in states]


def _cat_states(parts):
    return [{k: torch.cat([p[l][k] for p in parts], 0) for k in parts[0][l]} for l in range(len(parts[0]))]


def grpo_rollout(sd, input_ids, max_new_tokens, num_generations, *, eos=None, max_valid_id=None,
                 temperature=0.0, top_p=1.0, top_k=0, caps=None, dtype=torch.float32, max_steps=None, gen=None):
    """Returns (tokens per path, number of decode steps run)."""
    uniq, prompt_of = [], []
    seen = {}
    for p in input_ids:
        key = tuple(p)
        if key not in seen:
            seen[key] = len(uniq)
            uniq.append(list(p))
        prompt_of.append(seen[key])
    pstates, plogits = [], []
    for p in uniq:
        lg, st = om.forward_with_state(sd, torch.tensor([p]), None, dtype)
        pstates.append(st)
        plogits.append(lg[0, -1])
    G = num_generations
    paths = [prompt_of[b] for b in range(len(input_ids)) for _ in range(G)]
    n = len(paths)
    cap = [max_new_tokens] * n if caps is None else list(caps)
    states = _cat_states([_fork(pstates[u], [0]) for u in paths])
    toks = [[_pick(plogits[u], temperature, top_p, top_k, max_valid_id, osm.RULE_SINGLE, gen)] for u in paths]
    live = list(range(n))
    steps = 0
    while live and (max_steps is None or steps < max_steps):
        x = torch.tensor([[toks[q][-1]] for q in live])
        sub = _fork(states, live)
        lg, sub = om.forward_with_state(sd, x, sub, dtype)
        for l in range(len(states)):
            for k in states[l]:
                states[l][k][live] = sub[l][k]
        picks = _batch_pick(lg[:, -1], temperature, top_p, top_k, max_valid_id, osm.RULE_BATCH, gen)
        nxt = []
        for q, t in zip(live, picks):
            toks[q].append(t)
            if not ((eos is not None and t == eos) or len(toks[q]) >= cap[q]):
                nxt.append(q)
        live = nxt
        steps += 1
    return toks, steps


def scheduler_rollout(sd, prompts, max_new_tokens, *, eos=None, max_valid_id=None, dtype=torch.float32):
    """Greedy, one sequence at a time (the per-sequence meaning of SchedulerCore)."""
    out = []
    for p in prompts:
        lg, st = om.forward_with_state(sd, torch.tensor([p]), None, dtype)
        toks = []
        while True:
            t = osm.greedy(lg[0, -1], max_valid_id)[0]
            toks.append(t)
            if (eos is not None and t == eos) or len(toks) >= max_new_tokens:
                break
            lg, st = om.forward_with_state(sd, torch.tensor([[t]]), st, dtype)
        out.append(toks)
    return out
