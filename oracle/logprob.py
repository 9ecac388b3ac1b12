"""CPU restatement of the reference's GRPO log-prob recompute (test
infrastructure; see ``oracle/__init__``).

``selective_log_softmax(logits, index)``
    ``rwkvtune/training/grpo/utils.py:13-103``: log_softmax(logits)[index]
    without the full log-softmax.  float32 / float64 logits: gathered logit
    minus ``torch.logsumexp`` (``:43-53``).  bf16 / fp16 logits: logsumexp in
    float32, cast back to the dtype, subtracted in the dtype (``:54-101``).
``build_inputs(prompt_ids, completion_ids, ctx_len)``
    the input construction of ``_compute_per_token_logps_with_model``
    (``rwkvtune/training/grpo/lightning_module.py:1870-1910``): prompt followed by
    completion[:-1], the prompt cut to ``ctx_len - (C - 1)`` tokens (its first
    ones are kept), then right zero-padding to a multiple of 16, or, when that
    would exceed ctx_len, truncation to the largest multiple of 16 <= ctx_len.
    Returns (input_ids, logits_to_keep, C).
``per_token_logps(sd, prompt_ids, completion_ids, ctx_len, dtype)``
    the whole recompute over the restated model (``oracle.model``): forward from
    a zero state, ln_out and head over the last ``logits_to_keep`` positions
    (``rwkvtune/models/rwkv7/model.py:435-466``), the first C of them, then
    ``selective_log_softmax``.

Pinning (tests/test_oracle_logprob.py): log_softmax identities (the
probabilities of all V indices sum to 1; shift invariance; uniform logits give
-log V; one dominant logit gives ~0), agreement with torch.log_softmax + gather,
the bf16 rounding rule on hand-made rows, and the input construction on
hand-worked shapes (no cut, prompt cut, padding, truncation).
"""

from __future__ import annotations

import torch

from . import model as om

CHUNK_LEN = 16  # lightning_module.py:1893


def selective_log_softmax(logits: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """grpo/utils.py:13-103 (the loop over the leading dimension changes nothing
    numerically, so rows are processed together)."""
    sel = torch.gather(logits, -1, index.unsqueeze(-1)).squeeze(-1)
    if logits.dtype in (torch.float32, torch.float64):
        return sel - torch.logsumexp(logits, dim=-1)
    lse = torch.logsumexp(logits.float(), dim=-1).to(logits.dtype)
    return sel - lse


def build_inputs(prompt_ids: torch.Tensor, completion_ids: torch.Tensor, ctx_len: int):
    """lightning_module.py:1870-1910."""
    B, P = prompt_ids.shape
    C = completion_ids.shape[1]
    completion_input = completion_ids[:, :-1]
    max_prompt_len = ctx_len - completion_input.shape[1]
    if P > max_prompt_len:
        prompt_ids = prompt_ids[:, :max_prompt_len]
        P = max_prompt_len
    input_ids = torch.cat([prompt_ids, completion_input], dim=1)
    seq_len = input_ids.shape[1]
    pad_len = 0
    if seq_len % CHUNK_LEN != 0:
        pad_len = CHUNK_LEN - (seq_len % CHUNK_LEN)
        if seq_len + pad_len > ctx_len:
            max_seq_len = (ctx_len // CHUNK_LEN) * CHUNK_LEN
            input_ids = input_ids[:, :max_seq_len]
            pad_len = 0
        else:
            input_ids = torch.cat([input_ids, torch.zeros(B, pad_len, dtype=input_ids.dtype)], dim=1)
    return input_ids, C + pad_len, C


def per_token_logps(sd, prompt_ids, completion_ids, ctx_len: int, dtype=torch.float64):
    """lightning_module.py:1810-1964 with batch_size=None, over the oracle model."""
    input_ids, keep, C = build_inputs(prompt_ids, completion_ids, ctx_len)
    T = input_ids.shape[1]
    logits, _ = om.forward_with_state(sd, input_ids, None, dtype)
    if keep < T:
        logits = logits[:, -keep:]
    logits = logits[:, :C]
    return selective_log_softmax(logits, completion_ids)
