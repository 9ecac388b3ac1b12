"""Device-side token sampling - the drop-in for ``rwkvtune/inference/core.py``
``TokenSampler`` - plus the batched entry point the rollout engine uses.

``TokenSampler.sample(logits [V], ...) -> (int, float)`` and
``TokenSampler.sample_batch(logits [B, V], ...) -> (tokens [B], logps [B])`` keep
the reference's signatures and rules (``core.py:40-137`` / ``:142-236``; the two
nucleus rules differ and both are kept).  ``TokenSampler._max_valid_token_id``
bans larger ids, as in the reference (``core.py:66-77``).

The work is two HIP kernels (``rwkv7_sample``): no sort of the vocabulary, no
host round trip inside a batch.  Random draws come from a counter-based hash of
``(seed, key, counter)`` instead of torch's generator, so sampled streams are
reproducible per sequence and position but not bit-identical to
``torch.multinomial``; the sampling distribution is the reference's.
``TokenSampler.manual_seed(s)`` resets the seed and the call counter.

``logits_processor`` (JSON-schema masking in the reference) is applied in torch
on the device before the kernel, after temperature and bias, as in the reference.
"""

from __future__ import annotations

import threading
from typing import Callable, Optional, Tuple

import torch

from . import _lib

RULE_BATCH = 0
RULE_SINGLE = 1
RULE_MIXIN = 2   # GenerationMixin.generate (generation_mixin.py:180-211)


class SamplerBuffers:
    """Per-row sampling parameters on the device, for ``sample_rows``."""

    def __init__(self, n: int, device):
        self.temperature = torch.ones(n, dtype=torch.float32, device=device)
        self.top_p = torch.ones(n, dtype=torch.float32, device=device)
        self.top_k = torch.zeros(n, dtype=torch.int32, device=device)
        self.rng_key = torch.zeros(n, dtype=torch.int64, device=device)
        self.rng_ctr = torch.zeros(n, dtype=torch.int32, device=device)
        self.bias_off = None
        self.bias_ids = None
        self.bias_val = None

    def set_uniform(self, temperature: float, top_p: float, top_k: int):
        self.temperature.fill_(float(temperature))
        self.top_p.fill_(float(top_p))
        self.top_k.fill_(int(top_k))

    def set_bias(self, logit_bias: Optional[dict], n_rows: int):
        """The same ``{token_id: bias}`` for every row (GRPO passes one dict)."""
        if not logit_bias:
            self.bias_off = self.bias_ids = self.bias_val = None
            return
        dev = self.temperature.device
        ids = [int(k) for k in logit_bias.keys()]
        vals = [float(v) for v in logit_bias.values()]
        n = len(ids)
        self.bias_ids = torch.tensor(ids * n_rows, dtype=torch.int32, device=dev)
        self.bias_val = torch.tensor(vals * n_rows, dtype=torch.float32, device=dev)
        self.bias_off = torch.arange(0, (n_rows + 1) * n, n, dtype=torch.int32, device=dev)


def sample_rows(logits: torch.Tensor, buf: SamplerBuffers, *, rule: int, max_valid_id: Optional[int],
                seed: int, out_tok: torch.Tensor, out_logp: torch.Tensor,
                active: Optional[torch.Tensor] = None, n_rows: Optional[int] = None):
    """Sample one token per row of ``logits [M, V]`` (float32 / bf16 / fp16) into
    ``out_tok`` (int64) and ``out_logp`` (float32); rows with ``active == 0`` are
    skipped.  Enqueued on the current stream; no synchronisation."""
    M = logits.shape[0] if n_rows is None else n_rows
    V = logits.shape[-1]
    if logits.stride(-1) != 1:
        raise RuntimeError("logits rows must be contiguous")
    P = _lib.ptr
    _lib.call("rwkv7_sample", _lib.dtype_code(logits.dtype), M, V, P(logits), logits.stride(0), rule,
              -1 if max_valid_id is None else int(max_valid_id), P(buf.temperature), P(buf.top_p),
              P(buf.top_k), P(buf.bias_off), P(buf.bias_ids), P(buf.bias_val), P(active),
              ctypes_u64(seed), P(buf.rng_key), P(buf.rng_ctr), P(out_tok), P(out_logp),
              _lib.stream_of(logits))


def ctypes_u64(x: int):
    import ctypes
    return ctypes.c_uint64(int(x) & 0xFFFFFFFFFFFFFFFF)


def repetition_penalty_(logits: torch.Tensor, penalty: float, hist: torch.Tensor, hist_start: torch.Tensor,
                        hist_len: torch.Tensor, hist2=None, hist2_start=None, hist2_len=None, active=None,
                        n_rows=None):
    """In-place repetition penalty on float32 ``logits [M, V]``; row m's history is
    ``hist[hist_start[m]:+hist_len[m]]`` then ``hist2[hist2_start[m]:+hist2_len[m]]``
    (``grpo_batch_generator.py:25-42``: every occurrence applies once)."""
    if penalty == 1.0 or penalty <= 0:
        return logits
    if logits.dtype != torch.float32:
        raise RuntimeError("repetition penalty works on float32 logits")
    M = logits.shape[0] if n_rows is None else n_rows
    P = _lib.ptr
    import ctypes
    _lib.call("rwkv7_repetition_penalty", M, logits.shape[-1], P(logits), logits.stride(0),
              ctypes.c_float(penalty), P(hist), P(hist_start), P(hist_len), P(hist2), P(hist2_start),
              P(hist2_len), P(active), _lib.stream_of(logits))
    return logits


class TokenSampler:
    """Drop-in for ``rwkvtune.inference.core.TokenSampler`` on the GPU."""

    _max_valid_token_id: Optional[int] = None
    _seed: int = 0x5EED
    _calls: int = 0
    _lock = threading.Lock()

    @classmethod
    def manual_seed(cls, seed: int):
        with cls._lock:
            cls._seed = int(seed)
            cls._calls = 0

    @classmethod
    def _next_key(cls) -> int:
        with cls._lock:
            cls._calls += 1
            return cls._calls

    @staticmethod
    def _prepare(logits, temperature, logit_bias, logits_processor):
        """With a logits processor, temperature / bias / processor run here in the
        reference's order and the kernel then sees temperature 1 and no bias."""
        if logits_processor is None or temperature == 0 or temperature < 1e-6:
            return logits, temperature, logit_bias
        x = logits.float()
        mv = TokenSampler._max_valid_token_id
        if mv is not None and mv + 1 < x.shape[-1]:
            x = x.clone()
            x[..., mv + 1:] = float("-inf")
        if temperature != 1.0:
            x = x / temperature
        if logit_bias:
            x = x.clone()
            for tid, bias in logit_bias.items():
                t = int(tid)
                if 0 <= t < x.shape[-1]:
                    x[..., t] += min(100.0, max(-100.0, bias))
        return logits_processor(x), 1.0, None

    @staticmethod
    def _run(logits2d, temperature, top_p, top_k, logit_bias, rule):
        if not logits2d.is_cuda:
            raise RuntimeError("TokenSampler runs on the GPU; logits must be a device tensor")
        logits2d = logits2d.contiguous()
        B = logits2d.shape[0]
        buf = SamplerBuffers(B, logits2d.device)
        buf.set_uniform(temperature, top_p, top_k)
        buf.set_bias(logit_bias, B)
        buf.rng_key.fill_(TokenSampler._next_key())
        buf.rng_ctr.copy_(torch.arange(B, dtype=torch.int32, device=logits2d.device))
        tok = torch.empty(B, dtype=torch.int64, device=logits2d.device)
        lp = torch.empty(B, dtype=torch.float32, device=logits2d.device)
        sample_rows(logits2d, buf, rule=rule, max_valid_id=TokenSampler._max_valid_token_id,
                    seed=TokenSampler._seed, out_tok=tok, out_logp=lp)
        return tok, lp

    @staticmethod
    def sample(logits: torch.Tensor, temperature: float = 1.0, top_p: float = 1.0, top_k: int = 0,
               logit_bias: Optional[dict] = None,
               logits_processor: Optional[Callable[[torch.Tensor], torch.Tensor]] = None) -> Tuple[int, float]:
        if logits.dim() != 1:
            raise ValueError(f"Single sample requires 1D logits, got shape {logits.shape}")
        x, t, bias = TokenSampler._prepare(logits, temperature, logit_bias, logits_processor)
        tok, lp = TokenSampler._run(x.unsqueeze(0), t, top_p, top_k, bias, RULE_SINGLE)
        return int(tok.item()), float(lp.item())

    @staticmethod
    def sample_batch(logits_batch: torch.Tensor, temperature: float = 1.0, top_p: float = 1.0,
                     top_k: int = 0, logit_bias: Optional[dict] = None,
                     logits_processor: Optional[Callable[[torch.Tensor], torch.Tensor]] = None
                     ) -> Tuple[torch.Tensor, torch.Tensor]:
        if logits_batch.dim() != 2:
            raise ValueError(f"Batch sampling requires 2D logits, got shape {logits_batch.shape}")
        x, t, bias = TokenSampler._prepare(logits_batch, temperature, logit_bias, logits_processor)
        return TokenSampler._run(x, t, top_p, top_k, bias, RULE_BATCH)
