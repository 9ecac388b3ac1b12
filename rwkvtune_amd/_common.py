"""Helpers shared by the rollout front ends."""

from __future__ import annotations

from typing import List, Optional, Sequence


def max_valid_token_id(tokenizer) -> Optional[int]:
    """Largest id the tokenizer can decode; ids above it are banned when sampling
    (``grpo_batch_generator.py:104-106``, ``scheduler_core.py:177-178``)."""
    idx = getattr(tokenizer, "idx2token", None)
    if idx:
        return max(idx.keys())
    return None


def decode_tokens(tokenizer, ids: Sequence[int]) -> str:
    """``tokenizer.decode`` with the reference's tolerant fallback
    (``grpo_batch_generator.py:684-712``); no tokenizer gives ""."""
    if tokenizer is None or len(ids) == 0:
        return ""
    try:
        return tokenizer.decode(list(ids))
    except (KeyError, UnicodeDecodeError):
        tok = getattr(tokenizer, "idx2token", None)
        if tok is None:
            return ""
        return b"".join(tok.get(t, b"?") for t in ids).decode("utf-8", errors="replace")


def dedupe(prompts: Sequence[Sequence[int]]):
    """Distinct prompts in first-seen order and the index of each input's prompt."""
    uniq, index, order = {}, [], []
    for p in prompts:
        key = tuple(int(t) for t in p)
        if key not in uniq:
            uniq[key] = len(order)
            order.append(list(key))
        index.append(uniq[key])
    return order, index
