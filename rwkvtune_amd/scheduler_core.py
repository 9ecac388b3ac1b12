"""``SchedulerCore`` - continuous batching over a slot pool - with the public
surface of ``rwkvtune/inference/scheduler_core.py``: ``SeqStatus``,
``SequenceState`` (``:38-108``), ``SchedulerCore(model, tokenizer,
max_batch_size, max_batch_tokens, prefill_chunk_size, state_cache)`` with
``add_sequences / add_sequence / has_pending_work / get_stats / reset /
step_sync / run_to_completion_sync / step_async`` (``:111-782``) and
``create_scheduler_core`` (``:789-815``).

Semantics kept: every sequence is prefilled in chunks of ``prefill_chunk_size``
tokens under a ``max_batch_tokens`` budget per forward, its first token comes
from the prefill logits and every token uses ``TokenSampler.sample`` rules with
the sequence's own temperature / top_p / top_k / logit_bias; a sequence finishes
on ``eos_token_id`` or after ``max_new_tokens`` tokens (the first token included,
``:90-108``), freeing its slot for the next waiting sequence; at most
``max_batch_size`` sequences decode together.

Execution differs: the waiting sequences of a call run as one device-resident
rollout (``rwkvtune_amd.engine``), so the per-step token lists that
``step_sync`` / ``run_to_completion_sync`` hand out are recorded on the GPU and
returned after it finishes rather than with a host round trip per step and per
sequence.  Sequences added while results are being handed out run in the next
call.  Identical prompts are prefilled once.  Stop strings, JSON-schema
enforcers and the prefix state cache are not supported (``stop`` is accepted and
ignored, ``enforcer`` / ``state_cache`` raise).
"""

from __future__ import annotations

import collections
from dataclasses import dataclass, field
from enum import Enum, auto
from typing import Any, Dict, Iterator, List, Optional, Tuple, Union

import torch

from ._common import dedupe, max_valid_token_id
from .engine import RolloutEngine
from .model import as_hip_model
from .sampler import RULE_SINGLE, TokenSampler


class SeqStatus(Enum):
    WAITING = auto()
    PREFILLING = auto()
    RUNNING = auto()
    FINISHED = auto()


@dataclass
class SequenceState:
    seq_id: Union[int, str]
    prompt_tokens: List[int]
    status: SeqStatus = SeqStatus.WAITING
    prefill_offset: int = 0
    generated_tokens: List[int] = field(default_factory=list)
    last_token_id: Optional[int] = None
    max_new_tokens: int = 256
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = 0
    logit_bias: Optional[dict] = None
    stop: List[str] = field(default_factory=list)
    eos_token_id: Optional[int] = None
    generated_text: str = ""
    slot_id: int = -1
    original_tokens: Optional[List[int]] = None
    cached_prefix_len: int = 0
    cached_state: Optional[Any] = None
    cached_output: Optional[torch.Tensor] = None
    output_queue: Optional[Any] = None
    enforcer: Optional[Any] = None
    enforcer_finished: bool = False
    generated_logps: List[float] = field(default_factory=list)

    @property
    def is_finished(self) -> bool:
        if self.enforcer is not None and self.enforcer_finished:
            return True
        if self.eos_token_id is not None and self.last_token_id == self.eos_token_id:
            return True
        return len(self.generated_tokens) >= self.max_new_tokens


class SchedulerCore:
    def __init__(self, model, tokenizer, max_batch_size: int = 64, max_batch_tokens: int = 8192,
                 prefill_chunk_size: int = 512, state_cache=None):
        if state_cache is not None:
            raise NotImplementedError("the prefix state cache is not part of rwkvtune_amd")
        self.model = model
        self._hip = as_hip_model(model)
        self.tokenizer = tokenizer
        self.device = next(model.parameters()).device
        self.dtype = next(model.parameters()).dtype
        self.max_batch_size = max_batch_size
        self.max_batch_tokens = max_batch_tokens
        self.prefill_chunk_size = prefill_chunk_size
        self.state_cache = None
        self.n_layer = self._hip.config.n_layer
        self.n_embd = self._hip.config.n_embd
        self.head_size = 64
        self.n_head = self.n_embd // self.head_size
        self.sampler = TokenSampler
        mv = max_valid_token_id(tokenizer)
        if mv is not None:
            TokenSampler._max_valid_token_id = mv
        self._engine: Optional[RolloutEngine] = None
        self._calls = 0
        self.reset()

    # -- queues ----------------------------------------------------------------

    def reset(self) -> None:
        self.waiting_queue: collections.deque = collections.deque()
        self.prefilling_seqs: List[SequenceState] = []
        self.running_seqs: List[SequenceState] = []
        self.slots: List[Optional[SequenceState]] = [None] * self.max_batch_size
        self.free_slots = collections.deque(range(self.max_batch_size))
        self._pending_steps: collections.deque = collections.deque()

    def add_sequences(self, sequences: List[SequenceState]) -> None:
        for s in sequences:
            self.add_sequence(s)

    def add_sequence(self, seq: SequenceState) -> None:
        if seq.enforcer is not None:
            raise NotImplementedError("JSON-schema enforcers are not supported")
        self.waiting_queue.append(seq)

    def has_pending_work(self) -> bool:
        return bool(self.waiting_queue or self.running_seqs or self._pending_steps)

    def get_stats(self) -> Dict[str, int]:
        return {"waiting": len(self.waiting_queue), "prefilling": len(self.prefilling_seqs),
                "running": len(self.running_seqs), "free_slots": len(self.free_slots)}

    # -- execution --------------------------------------------------------------

    def _run_waiting(self) -> None:
        """Roll out every waiting sequence on the device and queue the per-step
        token lists they produced."""
        seqs = list(self.waiting_queue)
        self.waiting_queue.clear()
        if not seqs:
            return
        # one device rollout per distinct (eos, logit_bias): both are per-run settings
        groups = collections.OrderedDict()
        for s in seqs:
            if len(s.prompt_tokens) == 0:
                raise ValueError(f"sequence {s.seq_id} has an empty prompt")
            key = (s.eos_token_id, tuple(sorted((int(k), float(v)) for k, v in (s.logit_bias or {}).items())))
            groups.setdefault(key, []).append(s)
        per_step = collections.defaultdict(list)
        slots = max(1, min(self.max_batch_size, 1024))
        for (eos, bias), group in groups.items():
            eng = RolloutEngine(self._hip, min(slots, len(group)), eos_token_id=eos,
                                max_valid_id=TokenSampler._max_valid_token_id)
            uniq, index = dedupe([s.prompt_tokens for s in group])
            for s in group:
                s.status = SeqStatus.RUNNING
            self.running_seqs.extend(group)
            res = eng.run(uniq, index, [s.max_new_tokens for s in group],
                          logit_bias=dict(bias) if bias else None, first_rule=RULE_SINGLE,
                          decode_rule=RULE_SINGLE, first_can_finish=True, chunk_size=self.prefill_chunk_size,
                          max_batch_tokens=self.max_batch_tokens,
                          per_seq_sampling=([s.temperature for s in group], [s.top_p for s in group],
                                            [s.top_k for s in group]),
                          seed=TokenSampler._seed * 7919 + self._calls)
            self._calls += 1
            for s, toks, lps, steps in zip(group, res.tokens, res.logps, res.steps):
                for t, lp, st in zip(toks, lps, steps):
                    per_step[st].append((s, t, lp))
        for st in sorted(per_step):
            self._pending_steps.append(per_step[st])

    def step_sync(self) -> List[Tuple[Union[int, str], int]]:
        """New tokens of the next step: ``[(seq_id, token_id), ...]``."""
        with torch.no_grad():
            if not self._pending_steps and self.waiting_queue:
                self._run_waiting()
            if not self._pending_steps:
                return []
            out = []
            for s, t, lp in self._pending_steps.popleft():
                s.last_token_id = t
                s.generated_tokens.append(t)
                s.generated_logps.append(lp)
                s.prefill_offset = len(s.prompt_tokens)
                out.append((s.seq_id, t))
                if s.is_finished:
                    s.status = SeqStatus.FINISHED
                    if s in self.running_seqs:
                        self.running_seqs.remove(s)
            return out

    def run_to_completion_sync(self) -> Iterator[List[Tuple[Union[int, str], int]]]:
        while self.has_pending_work():
            new = self.step_sync()
            if new:
                yield new
            elif not self._pending_steps and not self.waiting_queue:
                # nothing left to hand out: sequences still marked running ended
                # without a terminating token (cannot happen with a finite cap)
                for s in list(self.running_seqs):
                    s.status = SeqStatus.FINISHED
                self.running_seqs.clear()

    async def step_async(self):
        return self.step_sync()


def create_scheduler_core(model, tokenizer, max_batch_size: int = 64, max_batch_tokens: int = 8192,
                          prefill_chunk_size: int = 512, state_cache=None) -> SchedulerCore:
    return SchedulerCore(model=model, tokenizer=tokenizer, max_batch_size=max_batch_size,
                         max_batch_tokens=max_batch_tokens, prefill_chunk_size=prefill_chunk_size,
                         state_cache=state_cache)
