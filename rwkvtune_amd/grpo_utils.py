"""GRPO log-prob recompute on the HIP library: the step after a rollout.

``selective_log_softmax(logits, index)``
    ``rwkvtune/training/grpo/utils.py:13-103`` (same name, arguments and
    per-dtype numerics) on ``rwkv7_selective_log_softmax``: one read of each
    logits row, no log-softmax tensor.
``compute_per_token_logps(model, prompt_ids, completion_ids, batch_size=None)``
    ``GRPOLightningModule._compute_per_token_logps_with_model``
    (``rwkvtune/training/grpo/lightning_module.py:1810-1964``): the same input
    construction (prompt + completion[:-1], ``ctx_len`` cut, padding to a
    multiple of 16) and the same result ``[B*G, C]`` in the model's dtype.  The
    reference materialises ``[B*G, C, V]`` logits (34 GB for 512 x 512 tokens of
    RWKV-7); here the forward returns the ln_out hidden states of the C needed
    positions only, and the head runs over row chunks of at most ``row_chunk``
    rows, each followed by the selective log-softmax, so at most ``row_chunk x V``
    logits exist at a time.  The forward is the model's own (chunked WKV prefill
    from a zero state, the recurrence of the reference's training kernel).
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from . import _lib

CHUNK_LEN = 16  # the reference's padding multiple (lightning_module.py:1893)


def selective_log_softmax(logits: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """log_softmax(logits)[..., index] in the logits' dtype (``grpo/utils.py:13-103``)."""
    if logits.device.type != "cuda":
        raise RuntimeError("selective_log_softmax runs on the HIP library only; move the logits to a GPU")
    if index.shape != logits.shape[:-1]:
        raise RuntimeError(f"index shape {tuple(index.shape)} does not match logits {tuple(logits.shape)}")
    V = logits.shape[-1]
    x = logits.reshape(-1, V)
    if x.stride(-1) != 1:
        x = x.contiguous()
    idx = index.reshape(-1).to(device=logits.device, dtype=torch.int64).contiguous()
    out = torch.empty(x.shape[0], dtype=logits.dtype, device=logits.device)
    _lib.call("rwkv7_selective_log_softmax", _lib.dtype_code(logits.dtype), x.shape[0], V, _lib.ptr(x),
              x.stride(0), _lib.ptr(idx), _lib.ptr(out), _lib.stream_of(out))
    return out.view(index.shape)


def _build_inputs(prompt_ids: torch.Tensor, completion_ids: torch.Tensor, ctx_len: int):
    """The input construction of lightning_module.py:1870-1910: returns
    (input_ids [B, T], logits_to_keep, C)."""
    B, P = prompt_ids.shape
    C = completion_ids.shape[1]
    completion_input = completion_ids[:, :-1]
    max_prompt_len = ctx_len - completion_input.shape[1]
    if P > max_prompt_len:
        prompt_ids = prompt_ids[:, :max_prompt_len]
    input_ids = torch.cat([prompt_ids, completion_input], dim=1)
    seq_len = input_ids.shape[1]
    pad_len = 0
    if seq_len % CHUNK_LEN != 0:
        pad_len = CHUNK_LEN - (seq_len % CHUNK_LEN)
        if seq_len + pad_len > ctx_len:
            input_ids = input_ids[:, :(ctx_len // CHUNK_LEN) * CHUNK_LEN]
            pad_len = 0
        else:
            pad = torch.zeros(B, pad_len, dtype=input_ids.dtype, device=input_ids.device)
            input_ids = torch.cat([input_ids, pad], dim=1)
    return input_ids, C + pad_len, C


@torch.no_grad()
def compute_per_token_logps(model, prompt_ids: torch.Tensor, completion_ids: torch.Tensor,
                            batch_size: Optional[int] = None, row_chunk: int = 8192,
                            max_forward_tokens: int = 1 << 17) -> torch.Tensor:
    """Per-token log-probabilities ``[B*G, C]`` of ``completion_ids`` given
    ``prompt_ids`` under ``model`` (an ``rwkvtune_amd`` ``RWKV7Model``), as
    ``lightning_module.py:1810-1964`` computes them.  ``batch_size`` caps the
    sequences per forward as in the reference; forwards are further capped at
    ``max_forward_tokens`` tokens (activation memory).  Sequences are independent,
    so the split does not change the result."""
    dev = model.device
    prompt_ids = prompt_ids.to(dev)
    completion_ids = completion_ids.to(dev)
    if prompt_ids.shape[0] != completion_ids.shape[0]:
        raise ValueError(f"Batch size mismatch: prompt_ids {tuple(prompt_ids.shape)}, "
                         f"completion_ids {tuple(completion_ids.shape)}")
    BG = prompt_ids.shape[0]
    input_ids, keep, C = _build_inputs(prompt_ids, completion_ids, model.config.ctx_len)
    T = input_ids.shape[1]
    if T > model.config.ctx_len:
        raise AssertionError(f"Sequence length {T} exceeds max length {model.config.ctx_len}")
    # positions whose logits are used: the last `keep` of the padded sequence, of
    # which the first C (model.py:460-463 and lightning_module.py:1918-1920)
    first = max(T - keep, 0)
    used = min(C, T - first)
    if used < C:
        # the reference's gather then fails on the shape mismatch
        raise RuntimeError(f"only {used} logits positions for {C} completion tokens")
    step = BG if batch_size is None else max(1, int(batch_size))
    step = max(1, min(step, max_forward_tokens // T))
    out = torch.empty((BG, C), dtype=model.dtype, device=dev)
    head = model.head.weight
    for s0 in range(0, BG, step):
        s1 = min(BG, s0 + step)
        nb = s1 - s0
        pos = torch.arange(first, first + C, device=dev)
        rows = (torch.arange(nb, device=dev)[:, None] * T + pos[None, :]).reshape(-1).to(torch.int32)
        hidden = model.forward_hidden(input_ids[s0:s1], rows)          # [nb * C, n_embd]
        tgt = completion_ids[s0:s1].reshape(-1)
        res = out[s0:s1].view(-1)
        for r0 in range(0, hidden.shape[0], row_chunk):
            r1 = min(hidden.shape[0], r0 + row_chunk)
            logits = F.linear(hidden[r0:r1], head)
            res[r0:r1] = selective_log_softmax(logits, tgt[r0:r1])
    return out
