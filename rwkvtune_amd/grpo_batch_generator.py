"""``GRPOBatchGenerator``: the rollout ``GRPOTrainer`` calls
(``rwkvtune/training/grpo/lightning_module.py:743-787``), with the constructor,
``generate`` signature and returned dict of
``rwkvtune/inference/grpo_batch_generator.py:63-151, 680-748``.

Semantics kept from the reference:
  * identical prompts are prefilled once and their state is forked to every
    generation path (``:152-260``);
  * the first token of every path is drawn from its prompt's last logits with
    ``TokenSampler.sample`` rules (``:262-310``); decode tokens with
    ``TokenSampler.sample_batch`` rules (``:594``);
  * a path ends when it emits ``eos_token_id`` or has ``max_new_tokens`` tokens;
    the first token never ends a path (the reference marks it but keeps decoding,
    ``:283-285`` vs ``:466-471``), so ``max_new_tokens = 1`` yields 2 tokens, as there;
  * ids above the tokenizer's largest id are banned; repetition penalty applies
    to prompt + generated ids, once per occurrence (``:25-42``);
  * results: ``completions`` (decoded strings), ``completion_ids`` (LongTensor
    ``[B*G, max_len]``, 0-padded, on the model's device), ``masks`` (bool).

``model`` may be an ``rwkvtune_amd.RWKV7Model`` or any module with the
reference model's parameter names - the trainer's own model: its parameters
are used in place (``as_hip_model``) and parameter updates between calls are
picked up without any call from the trainer.

Differences, on purpose: decoding runs on the GPU slot table
(``rwkvtune_amd.engine``) with ``max_decode_batch_size`` slots (all paths when
-1, capped at 1024) and continuous refill instead of a shrinking lockstep batch;
prompts are prefilled ragged in one packed batch (``chunk_size`` tokens per
prompt per pass, ``max_prefill_batch_size`` prompts per forward); random draws
come from the engine's counter-based stream (set ``seed``); the reference's
``max_prefill_batch_size`` bug that re-runs the last prompt token
(``:405-421, 286-310``) is not reproduced.  ``max_new_tokens_per_seq`` (one cap
per path) is an addition used for forced stop lengths.
"""

from __future__ import annotations

import time
from typing import Any, Dict, List, Optional, Sequence

import torch

from ._common import decode_tokens, dedupe, max_valid_token_id
from .engine import RolloutEngine
from .model import as_hip_model
from .sampler import RULE_BATCH, RULE_SINGLE, TokenSampler


class GRPOBatchGenerator:
    def __init__(self, model, tokenizer, chunk_size: int = 2048, max_prefill_batch_size: int = -1,
                 max_decode_batch_size: int = -1, eos_token_id: Optional[int] = None, *, verbose: bool = True,
                 keep_decode_context: bool = True):
        self.model = model
        # False: release the decode context (slot pool, prompt store, graphs)
        # after every generate, so the trainer's forward / backward can use the memory
        self.keep_decode_context = keep_decode_context
        # the caller's module (e.g. GRPOTrainer's training model) runs through a
        # wrapper that shares its parameters; packed copies follow their updates
        self._hip = as_hip_model(model)
        self.tokenizer = tokenizer
        self.device = next(model.parameters()).device
        self.dtype = next(model.parameters()).dtype
        self.chunk_size = chunk_size
        self.max_prefill_batch_size = max_prefill_batch_size
        self.max_decode_batch_size = max_decode_batch_size
        self.eos_token_id = eos_token_id
        self.sampler = TokenSampler
        self.n_layer = self._hip.config.n_layer
        self.n_embd = self._hip.config.n_embd
        self.verbose = verbose
        mv = max_valid_token_id(tokenizer)
        if mv is not None:
            TokenSampler._max_valid_token_id = mv
        self._engines = {}
        self._calls = 0
        self.last_stats: Dict[str, Any] = {}

    def _engine(self, slots: int) -> RolloutEngine:
        eng = self._engines.get(slots)
        if eng is None:
            eng = RolloutEngine(self._hip, slots, eos_token_id=self.eos_token_id,
                                max_valid_id=TokenSampler._max_valid_token_id)
            self._engines = {slots: eng}
        return eng

    @torch.no_grad()
    def generate(self, input_ids: List[List[int]], max_new_tokens: int, num_generations: int = 1,
                 temperature: float = 0.9, top_p: float = 0.9, top_k: int = 0, repetition_penalty: float = 1.0,
                 logit_bias: Optional[dict] = None, *, max_new_tokens_per_seq: Optional[Sequence[int]] = None,
                 seed: Optional[int] = None) -> Dict[str, Any]:
        # the trainer may have replaced parameters (or wrapped linears with LoRA)
        # since the last call: re-bind the same wrapper to its current ones
        self._hip = as_hip_model(self.model)
        B = len(input_ids)
        G = num_generations
        total = B * G
        uniq, prompt_of = dedupe(input_ids)
        seq_prompt = [prompt_of[b] for b in range(B) for _ in range(G)]
        if max_new_tokens_per_seq is not None:
            if len(max_new_tokens_per_seq) != total:
                raise ValueError("max_new_tokens_per_seq needs one entry per generation path")
            caps = [max(1, min(int(c), max_new_tokens)) for c in max_new_tokens_per_seq]
        else:
            caps = max_new_tokens
        slots = self.max_decode_batch_size if self.max_decode_batch_size > 0 else total
        slots = max(1, min(slots, total, 1024))
        eng = self._engine(slots)
        if seed is None:
            seed = TokenSampler._seed * 1000003 + self._calls
        self._calls += 1
        t0 = time.time()
        res = eng.run(uniq, seq_prompt, caps, temperature=temperature, top_p=top_p, top_k=top_k,
                      logit_bias=logit_bias, repetition_penalty=repetition_penalty, first_rule=RULE_SINGLE,
                      decode_rule=RULE_BATCH, first_can_finish=False, chunk_size=self.chunk_size,
                      max_seqs_per_forward=max(0, self.max_prefill_batch_size), seed=seed)
        if not self.keep_decode_context:
            eng.release()
        wall = time.time() - t0
        gen = sum(res.ngen)
        tm = res.timings
        # the reference's own throughput definitions (grpo_batch_generator.py:327-349)
        self.last_stats = {
            "unique_prompts": len(uniq), "total_sequences": total, "prompt_tokens": res.prompt_tokens,
            "generated_tokens": gen, "decode_steps": res.n_decode_steps, "wall_s": wall, **tm,
            "decode_throughput": gen / tm["decode_s"] if tm.get("decode_s") else 0.0,
            "overall_throughput": (res.prompt_tokens + gen) / wall if wall > 0 else 0.0,
        }
        if self.verbose:
            print(f"[GRPOBatchGenerator] {total} sequences ({len(uniq)} unique prompts, "
                  f"{res.prompt_tokens} prompt tokens): generated {gen} tokens in {res.n_decode_steps} decode "
                  f"steps; prefill {tm['prefill_s']:.3f}s, decode {tm['decode_s']:.3f}s, total {wall:.3f}s")
        return self._collect_results(res)

    def release(self):
        """Free the decode contexts kept for the next call (see ``RolloutEngine.release``)."""
        for eng in self._engines.values():
            eng.release()

    def _collect_results(self, res) -> Dict[str, Any]:
        """completions (decoded text), completion_ids ``[total, L]`` (zero past each
        sequence's end) and masks, as the reference returns them
        (``grpo_batch_generator.py:680-750``)."""
        ids, masks = res.padded_ids()
        if self.tokenizer is None:
            completions = [""] * len(res.ngen)
        else:
            completions = [decode_tokens(self.tokenizer, t) for t in res.tokens]
        return {"completions": completions, "completion_ids": ids.to(self.device),
                "masks": masks.to(self.device)}
