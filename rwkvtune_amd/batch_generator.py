"""``BatchGenerator`` / ``GenerationConfig``: the synchronous batch front end of
``rwkvtune/inference/batch_generator.py:28-244`` over ``SchedulerCore``.

Kept: G copies of each prompt (``:106-111``), at most
``config.generation_max_batch_size`` (default 256) concurrent sequences, a
trailing EOS stripped from each completion (``:199-202``), and the result dict
``completions``, ``completion_ids`` (LongTensor, 0-padded), ``completion_logps``
(empty tensor), ``masks`` (float32, as the reference returns).
``use_state_cache=True`` is accepted with a warning and ignored: the prefix
state cache only skips recomputation, results are unchanged.
"""

from __future__ import annotations

import warnings
from dataclasses import dataclass
from typing import Any, Dict, List, Optional

import torch

from ._common import decode_tokens
from .scheduler_core import SequenceState, SeqStatus, create_scheduler_core

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
        self._scheduler = None

    def generate(self, prompts: Optional[List[str]] = None, generation_config: GenerationConfig = None,
                 input_ids: Optional[List[List[int]]] = None) -> Dict[str, Any]:
        if generation_config is None:
            generation_config = GenerationConfig()
        if input_ids is None:
            if prompts is None:
                raise ValueError("Must provide prompts or input_ids")
            input_ids = [self.tokenizer.encode(p) for p in prompts]
        G = generation_config.num_generations
        expanded = [list(ids) for ids in input_ids for _ in range(G)]
        total = len(expanded)
        max_batch = max(1, min(getattr(self.config, "generation_max_batch_size", 256), total))
        sch = self._scheduler
        if (sch is None or sch.max_batch_size != max_batch
                or sch.max_batch_tokens != generation_config.max_batch_tokens
                or sch.prefill_chunk_size != generation_config.chunk_size):
            sch = self._scheduler = create_scheduler_core(
                self.model, self.tokenizer, max_batch_size=max_batch,
                max_batch_tokens=generation_config.max_batch_tokens, prefill_chunk_size=generation_config.chunk_size)
        else:
            sch.reset()
        seqs = [SequenceState(seq_id=i, prompt_tokens=t, max_new_tokens=generation_config.max_length,
                              temperature=generation_config.temperature, top_p=generation_config.top_p,
                              top_k=generation_config.top_k, eos_token_id=self.eos_id)
                for i, t in enumerate(expanded)]
        sch.add_sequences(seqs)
        all_tokens: List[List[int]] = [[] for _ in range(total)]
        for updates in sch.run_to_completion_sync():
            for sid, tok in updates:
                all_tokens[sid].append(tok)
        return self._postprocess(all_tokens, total)

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
