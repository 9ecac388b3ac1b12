"""``BatchGenerator`` / ``GenerationConfig``: the synchronous batch front end of
``rwkvtune/inference/batch_generator.py:28-244``.

Kept: G copies of each prompt (``:106-111``), each prefilled (no dedupe), at
most ``config.generation_max_batch_size`` (default 256) concurrent sequences,
``GenerationConfig.chunk_size`` prompt tokens per sequence and
``max_batch_tokens`` per prefill forward, ``TokenSampler.sample`` rules for every
token (the reference runs ``SchedulerCore``, ``scheduler_core.py:470-476,
563-569``), a trailing EOS stripped from each completion (``:199-202``), and the
result dict ``completions``, ``completion_ids`` (LongTensor, 0-padded),
``completion_logps`` (empty tensor), ``masks`` (float32, as the reference
returns).  ``use_state_cache=True`` is accepted with a warning and ignored: the
prefix state cache only skips recomputation, results are unchanged.

The whole batch runs on the rollout engine's slot table with the prompts
prefilled in their slots (``RolloutEngine.run_inline``): finished sequences
retire and waiting ones are admitted into the freed slots on the device, and no
decode step waits for the host.  Random draws come from the engine's
(sequence, position) streams (``seed``); ``max_new_tokens_per_seq`` (one cap per
sequence) is an addition used for forced stop lengths.
"""

from __future__ import annotations

import warnings
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Sequence

import torch

from ._common import decode_tokens, max_valid_token_id
from .engine import RolloutEngine
from .model import as_hip_model
from .sampler import RULE_SINGLE, TokenSampler
from .scheduler_core import SeqStatus

ReqStatus = SeqStatus


@dataclass
class GenerationConfig:
    max_length: int = 256
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = 0
    num_generations: int = 1
    max_batch_tokens: int = 8192
    chunk_size: int = 512


class BatchGenerator:
    def __init__(self, model, tokenizer, config=None, use_state_cache: bool = False, **kwargs):
        self.model = model
        self.tokenizer = tokenizer
        self.config = config
        self.device = next(model.parameters()).device
        self.eos_id = getattr(tokenizer, "eos_token_id", None)
        if use_state_cache:
            warnings.warn("rwkvtune_amd has no prefix state cache; generating without it")
        self.state_cache = None
        mv = max_valid_token_id(tokenizer)
        if mv is not None:
            TokenSampler._max_valid_token_id = mv
        self._engines: Dict[int, RolloutEngine] = {}
        self.last_stats: Dict[str, Any] = {}

    def _engine(self, slots: int) -> RolloutEngine:
        hip = as_hip_model(self.model)
        eng = self._engines.get(slots)
        if eng is None or eng.model is not hip:
            eng = RolloutEngine(hip, slots, eos_token_id=self.eos_id, max_valid_id=TokenSampler._max_valid_token_id)
            self._engines = {slots: eng}
        return eng

    def release(self):
        """Free the decode context kept for the next call (``RolloutEngine.release``)."""
        for eng in self._engines.values():
            eng.release()

    @torch.no_grad()
    def generate(self, prompts: Optional[List[str]] = None, generation_config: GenerationConfig = None,
                 input_ids: Optional[List[List[int]]] = None, *,
                 max_new_tokens_per_seq: Optional[Sequence[int]] = None, seed: Optional[int] = None
                 ) -> Dict[str, Any]:
        if generation_config is None:
            generation_config = GenerationConfig()
        if input_ids is None:
            if prompts is None:
                raise ValueError("Must provide prompts or input_ids")
            input_ids = [self.tokenizer.encode(p) for p in prompts]
        G = generation_config.num_generations
        expanded = [list(ids) for ids in input_ids for _ in range(G)]
        total = len(expanded)
        if total == 0:
            return self._postprocess([], 0)
        max_batch = max(1, min(getattr(self.config, "generation_max_batch_size", 256), total, 1024))
        caps = generation_config.max_length
        if max_new_tokens_per_seq is not None:
            if len(max_new_tokens_per_seq) != total:
                raise ValueError("max_new_tokens_per_seq needs one entry per sequence")
            caps = [max(1, min(int(c), generation_config.max_length)) for c in max_new_tokens_per_seq]
        if seed is None:
            seed = TokenSampler._seed * 7919 + TokenSampler._next_key()
        eng = self._engine(max_batch)
        res = eng.run_inline(expanded, caps, temperature=generation_config.temperature,
                             top_p=generation_config.top_p, top_k=generation_config.top_k,
                             first_rule=RULE_SINGLE, decode_rule=RULE_SINGLE,
                             chunk_size=generation_config.chunk_size,
                             max_batch_tokens=generation_config.max_batch_tokens, seed=seed)
        gen = sum(res.ngen)
        tm = res.timings
        self.last_stats = {"total_sequences": total, "prompt_tokens": res.prompt_tokens, "generated_tokens": gen,
                           "decode_steps": res.n_decode_steps, **tm}
        return self._postprocess([list(t) for t in res.tokens], total)

    def _postprocess(self, all_tokens: List[List[int]], total: int) -> Dict[str, Any]:
        completions = []
        for i, toks in enumerate(all_tokens):
            if self.eos_id is not None and toks and toks[-1] == self.eos_id:
                all_tokens[i] = toks = toks[:-1]
            completions.append(decode_tokens(self.tokenizer, toks))
        max_len = max((len(t) for t in all_tokens), default=0)
        if max_len > 0:
            ids = torch.zeros((total, max_len), dtype=torch.long)
            masks = torch.zeros((total, max_len), dtype=torch.float32)
            for i, t in enumerate(all_tokens):
                if t:
                    ids[i, :len(t)] = torch.tensor(t, dtype=torch.long)
                    masks[i, :len(t)] = 1.0
        else:
            ids = torch.zeros((total, 0), dtype=torch.long)
            masks = torch.zeros((total, 0), dtype=torch.float32)
        return {"completions": completions, "completion_ids": ids.to(self.device),
                "completion_logps": torch.tensor([], device=self.device), "masks": masks.to(self.device)}
