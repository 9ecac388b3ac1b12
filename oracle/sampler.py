"""CPU restatement of the reference's sampling rules (test infrastructure; see
``oracle/__init__``).  Follows ``rwkvtune/inference/core.py``:

``distribution(...)``  the exact distribution a call samples from, float64 [V]:
    RULE_SINGLE = ``TokenSampler.sample`` (``core.py:40-137``): ban ids above
    max_valid_id, temperature, logit_bias (clamped to +-100), softmax; top_k > 0
    keeps the k most probable and renormalises; else top_p < 1 keeps the sorted
    prefix of length #(cumsum <= p) + 1 (``:119-131``); non-finite probabilities
    give the uniform distribution (``:102-108``).
    RULE_BATCH = ``TokenSampler.sample_batch`` (``core.py:142-236``): top_k keeps
    the k largest logits, then top_p keeps the sorted prefix with cumsum <= p and
    always the first entry (``:214-228``); softmax over what is kept.
    RULE_MIXIN = ``GenerationMixin.generate`` (``rwkvtune/models/generation_mixin.py:
    180-211``): softmax; top_k > 0 keeps the k most probable and renormalises;
    then, only when 0 < top_p < 1, the sorted entries whose preceding cumulative
    sum is <= p (the shifted ``cumsum > p`` mask: the crossing entry is kept, the
    first always) and renormalises.  No id ban (the caller passes none).
``logp(...)``          the log-probability the reference returns for a token.
``greedy(...)``        argmax of the banned logits (first index on ties) and its
    log_softmax (``core.py:80-83, 184-188``).
Sorting is a stable descending sort by logit (ties by index).

Pinning (tests/test_oracle_sampler.py): hand-computed distributions on tiny
vocabularies for each rule (the single rule keeps exactly one more token than the
batch rule when the boundary is not the first token; top_k / top_p / both; ban and
bias), brute-force enumeration of the nucleus rule over random tiny rows, and the
normalisation of every returned distribution.
"""

from __future__ import annotations

import torch

RULE_BATCH = 0
RULE_SINGLE = 1
RULE_MIXIN = 2


def _prep(logits, temperature, logit_bias, max_valid_id):
    x = logits.detach().to(torch.float64).cpu().clone()
    if max_valid_id is not None and max_valid_id + 1 < x.shape[-1]:
        x[max_valid_id + 1:] = float("-inf")
    if temperature != 1.0:
        x = x / temperature
    if logit_bias:
        for tid, b in logit_bias.items():
            t = int(tid)
            if 0 <= t < x.shape[-1]:
                x[t] += min(100.0, max(-100.0, b))
    return x


def distribution(logits, temperature=1.0, top_p=1.0, top_k=0, logit_bias=None,
                 max_valid_id=None, rule=RULE_BATCH):
    x = _prep(logits, temperature, logit_bias, max_valid_id)
    V = x.shape[-1]
    order = torch.sort(-x, stable=True).indices  # descending, ties by index
    if rule == RULE_MIXIN:
        probs = torch.softmax(x, -1)
        if top_k > 0:
            kept = torch.zeros(V, dtype=torch.float64)
            kept[order[:min(top_k, V)]] = probs[order[:min(top_k, V)]]
            probs = kept / kept.sum()
        if 0.0 < top_p < 1.0:
            o2 = torch.sort(-probs, stable=True).indices
            cs = torch.cumsum(probs[o2], 0)
            remove = torch.zeros(V, dtype=torch.bool)
            remove[1:] = cs[:-1] > top_p
            kept = probs.clone()
            kept[o2[remove]] = 0.0
            probs = kept / kept.sum()
        return probs
    if rule == RULE_SINGLE:
        probs = torch.softmax(x, -1)
        if not torch.isfinite(probs).all():
            return torch.full((V,), 1.0 / V, dtype=torch.float64)
        keep = torch.zeros(V, dtype=torch.bool)
        if top_k > 0:
            keep[order[:min(top_k, V)]] = True
        elif top_p < 1.0:
            cs = torch.cumsum(probs[order], 0)
            cutoff = max(1, int((cs <= top_p).sum()) + 1)
            keep[order[:cutoff]] = True
        else:
            keep[:] = True
        out = torch.where(keep, probs, torch.zeros_like(probs))
        return out / out.sum()
    keep = torch.ones(V, dtype=torch.bool)
    if top_k > 0:
        keep[:] = False
        keep[order[:min(top_k, V)]] = True
    if top_p < 1.0:
        xm = torch.where(keep, x, torch.full_like(x, float("-inf")))
        order2 = torch.sort(-xm, stable=True).indices
        cs = torch.cumsum(torch.softmax(xm[order2], -1), 0)
        mask = cs <= top_p
        mask[0] = True
        keep2 = torch.zeros(V, dtype=torch.bool)
        keep2[order2[mask]] = True
        keep = keep & keep2
    xm = torch.where(keep, x, torch.full_like(x, float("-inf")))
    return torch.softmax(xm, -1)


def logp(dist, token, rule):
    p = float(dist[token])
    if rule in (RULE_SINGLE, RULE_MIXIN):
        return float(torch.log(torch.tensor(p + 1e-10, dtype=torch.float64)))
    return float(torch.log(torch.tensor(p, dtype=torch.float64)))


def greedy(logits, max_valid_id=None):
    x = _prep(logits, 1.0, None, max_valid_id)
    t = int(torch.argmax(x))
    return t, float(torch.log_softmax(x, -1)[t])


def repetition_penalty(logits, histories, penalty):
    """Row-wise, once per occurrence (``grpo_batch_generator.py:25-42``)."""
    out = logits.detach().to(torch.float64).cpu().clone()
    if penalty == 1.0 or penalty <= 0:
        return out
    for i, hist in enumerate(histories):
        for t in hist:
            if 0 <= t < out.shape[1]:
                out[i, t] = out[i, t] / penalty if out[i, t] > 0 else out[i, t] * penalty
    return out


def sample_batch_torch(logits, temperature=1.0, top_p=1.0, top_k=0, max_valid_id=None, gen=None):
    """Batched float32 restatement of ``TokenSampler.sample_batch``
    (``core.py:142-236``) in torch CPU ops, as the reference runs it on CPU: ban,
    temperature, top-k mask, sort + softmax + cumsum nucleus mask (first entry
    kept), restore order, softmax, multinomial, gathered log-softmax.  Used by
    the timed CPU baseline."""
    x = logits.float().clone()
    V = x.shape[1]
    if max_valid_id is not None and max_valid_id + 1 < V:
        x[:, max_valid_id + 1:] = float("-inf")
    if temperature == 0 or temperature < 1e-6:
        tok = x.argmax(-1)
        return tok, torch.log_softmax(x, -1).gather(1, tok[:, None])[:, 0]
    if temperature != 1.0:
        x = x / temperature
    if top_k > 0:
        vals, idx = torch.topk(x, top_k, dim=-1)
        x = torch.full_like(x, float("-inf")).scatter_(-1, idx, vals)
    if top_p < 1.0:
        sl, si = torch.sort(x, descending=True, dim=-1)
        cs = torch.cumsum(torch.softmax(sl, -1), -1)
        keep = cs <= top_p
        keep[:, 0] = True
        sl = sl.masked_fill(~keep, float("-inf"))
        _, restore = torch.sort(si, dim=-1)
        x = torch.gather(sl, -1, restore)
    tok = torch.multinomial(torch.softmax(x, -1), 1, generator=gen)[:, 0]
    return tok, torch.log_softmax(x, -1).gather(1, tok[:, None])[:, 0]
