"""``SchedulerCore`` - continuous batching over a slot pool - with the public
surface of ``rwkvtune/inference/scheduler_core.py``: ``SeqStatus``,
``SequenceState`` (``:38-108``), ``SchedulerCore(model, tokenizer,
max_batch_size, max_batch_tokens, prefill_chunk_size, state_cache)`` with
``add_sequences / add_sequence / has_pending_work / get_stats / reset /
step_sync / run_to_completion_sync / step_async`` (``:111-782``) and
``create_scheduler_core`` (``:789-815``).

One ``step_sync`` is one step of the reference's loop (``:250-299, 445-600,
606-664``):

1. admit waiting sequences into free slots (status PREFILLING) and zero those
   slots' state;
2. decode one token for every running sequence - one pooled single-token forward
   over their slots (rows addressed through the slot table, no gather / scatter
   of states) and one device sampler launch with each sequence's own
   temperature / top_p / top_k / logit_bias (``TokenSampler.sample`` rules),
   replayed as one captured graph per row bucket (rows with a logit_bias run
   eagerly);
3. prefill the next chunk (at most ``prefill_chunk_size`` tokens) of prefilling
   sequences under the ``max_batch_tokens`` budget, all chunks in one ragged
   forward (no grouping by length); a sequence whose prompt is complete draws its
   first token from the prefill logits and runs from the next step on;
4. a sequence finishes on ``eos_token_id`` or after ``max_new_tokens`` tokens
   (the first included, ``:90-108``) and frees its slot for the next admission.

The step returns its new ``(seq_id, token_id)`` pairs; sequences added between
steps are admitted as slots free up.  The slot pool (``max_batch_size`` slots,
float32 state) is allocated once, so memory does not grow with the queue.  The
step's one host synchronisation is the copy of the sampled ids.  Random draws
are keyed by (sequence, position), so a sequence's tokens do not depend on what
else is batched with it.  Stop strings, JSON-schema enforcers and the prefix
state cache are not supported (``stop`` is accepted and ignored, ``enforcer`` /
``state_cache`` raise).
"""

from __future__ import annotations

import collections
from dataclasses import dataclass, field
from enum import Enum, auto
from typing import Any, Dict, Iterator, List, Optional, Tuple, Union

import torch

from ._common import max_valid_token_id
from .engine import row_buckets
from .model import RWKV7Model, StatePool, as_hip_model
from .sampler import RULE_SINGLE, SamplerBuffers, TokenSampler, sample_rows


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


class _DecodeGraphs:
    """The decode step of a ``SchedulerCore`` on static row buffers, captured in
    one HIP graph per row bucket: rows 0 .. R-1 are the running sequences (their
    slot, input token and sampling inputs copied in before each replay from
    pinned host memory), rows R .. bucket-1 are inactive (slot -1).  A bucket's
    first step runs eagerly (lazy allocations happen outside capture), later
    ones replay its graph.  The graphs bake in the model's packed weights, the
    shared split-K workspace, the sampler's seed and id ban; a change of any of
    them drops them."""

    def __init__(self, S: int, dev):
        self.S = S
        self.tok = torch.zeros(S, dtype=torch.int64, device=dev)
        self.slot = torch.full((S,), -1, dtype=torch.int32, device=dev)
        self.last = torch.arange(S, dtype=torch.int32, device=dev)
        self.active = torch.zeros(S, dtype=torch.uint8, device=dev)
        self.buf = SamplerBuffers(S, dev)
        self.out_tok = torch.zeros(S, dtype=torch.int64, device=dev)
        self.out_lp = torch.zeros(S, dtype=torch.float32, device=dev)
        self.h_i64 = torch.zeros((2, S), dtype=torch.int64).pin_memory()    # token, random-stream key
        self.h_i32 = torch.zeros((3, S), dtype=torch.int32).pin_memory()    # slot, top_k, position
        self.h_f32 = torch.zeros((2, S), dtype=torch.float32).pin_memory()  # temperature, top_p
        self.h_u8 = torch.zeros(S, dtype=torch.uint8).pin_memory()          # active
        self.buckets = row_buckets(S)
        self.graphs = {}
        self.warm = set()
        self.graph_pool = torch.cuda.graph_pool_handle()
        self.key = None

    def load(self, batch):
        """Stage the rows of ``batch`` (running sequences) and copy them to the
        device on the current stream; returns the bucket to run."""
        R = len(batch)
        Mb = next(b for b in self.buckets if b >= R)
        self.h_i64.zero_()
        self.h_i32[0].fill_(-1)
        self.h_i32[1:].zero_()
        self.h_f32.fill_(1.0)
        self.h_u8.zero_()
        self.h_i64[0, :R] = torch.tensor([s.last_token_id for s in batch], dtype=torch.int64)
        self.h_i64[1, :R] = torch.tensor([s._rng_key for s in batch], dtype=torch.int64)
        self.h_i32[0, :R] = torch.tensor([s.slot_id for s in batch], dtype=torch.int32)
        self.h_i32[1, :R] = torch.tensor([int(s.top_k) for s in batch], dtype=torch.int32)
        self.h_i32[2, :R] = torch.tensor([len(s.generated_tokens) for s in batch], dtype=torch.int32)
        self.h_f32[0, :R] = torch.tensor([float(s.temperature) for s in batch], dtype=torch.float32)
        self.h_f32[1, :R] = torch.tensor([float(s.top_p) for s in batch], dtype=torch.float32)
        self.h_u8[:R] = 1
        for dst, src in ((self.tok, self.h_i64[0]), (self.buf.rng_key, self.h_i64[1]), (self.slot, self.h_i32[0]),
                         (self.buf.top_k, self.h_i32[1]), (self.buf.rng_ctr, self.h_i32[2]),
                         (self.buf.temperature, self.h_f32[0]), (self.buf.top_p, self.h_f32[1]),
                         (self.active, self.h_u8)):
            dst[:Mb].copy_(src[:Mb], non_blocking=True)
        return Mb

    def _body(self, hip, pool, Mb, seed, max_valid_id):
        logits = hip.forward_pooled(self.tok[:Mb], self.slot[:Mb], self.last[:Mb], pool, decode=True)
        sub = SamplerBuffers.__new__(SamplerBuffers)
        b = self.buf
        sub.temperature, sub.top_p, sub.top_k = b.temperature[:Mb], b.top_p[:Mb], b.top_k[:Mb]
        sub.rng_key, sub.rng_ctr = b.rng_key[:Mb], b.rng_ctr[:Mb]
        sub.bias_off = sub.bias_ids = sub.bias_val = None
        sample_rows(logits, sub, rule=RULE_SINGLE, max_valid_id=max_valid_id, seed=seed, out_tok=self.out_tok[:Mb],
                    out_logp=self.out_lp[:Mb], active=self.active[:Mb])

    def run(self, hip, pool, Mb, seed, max_valid_id):
        hip.packs()  # refresh the packed weights outside capture
        key = (hip._packs_gen, RWKV7Model.gemm_workspace(hip.device).ws.data_ptr(), seed, max_valid_id, id(pool))
        if key != self.key:
            self.graphs.clear()
            self.warm.clear()
            self.key = key
        g = self.graphs.get(Mb)
        if g is None and Mb in self.warm:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=self.graph_pool):
                self._body(hip, pool, Mb, seed, max_valid_id)
            self.graphs[Mb] = g
        if g is not None:
            g.replay()
        else:
            self._body(hip, pool, Mb, seed, max_valid_id)
            self.warm.add(Mb)


class SchedulerCore:
    def __init__(self, model, tokenizer, max_batch_size: int = 64, max_batch_tokens: int = 8192,
                 prefill_chunk_size: int = 512, state_cache=None):
        if state_cache is not None:
            raise NotImplementedError("the prefix state cache is not part of rwkvtune_amd")
        if max_batch_size < 1 or max_batch_size > 1024:
            raise ValueError("max_batch_size must be in [1, 1024]")
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
        # the slot pool: fixed size, whatever the queue length
        self.state_pool = StatePool(self._hip.config, max_batch_size, self.device)
        # decode steps replay a captured graph per row bucket (False: eager launches)
        self.use_graph = True
        self._graphs = _DecodeGraphs(max_batch_size, self.device)
        self._seed = TokenSampler._seed * 7919 + TokenSampler._next_key()
        self._keys = 0
        self._step_counter = 0
        self.reset()

    # -- queues ----------------------------------------------------------------

    def reset(self) -> None:
        """Clear the queues and free every slot (the state pool is kept)."""
        self.waiting_queue: collections.deque = collections.deque()
        self.prefilling_seqs: List[SequenceState] = []
        self.running_seqs: List[SequenceState] = []
        self.slots: List[Optional[SequenceState]] = [None] * self.max_batch_size
        self.free_slots = collections.deque(range(self.max_batch_size))

    def add_sequences(self, sequences: List[SequenceState]) -> None:
        for s in sequences:
            self.add_sequence(s)

    def add_sequence(self, seq: SequenceState) -> None:
        if seq.enforcer is not None:
            raise NotImplementedError("JSON-schema enforcers are not supported")
        if len(seq.prompt_tokens) == 0:
            raise ValueError(f"sequence {seq.seq_id} has an empty prompt")
        seq._rng_key = self._keys  # random stream of this sequence
        self._keys += 1
        self.waiting_queue.append(seq)

    def has_pending_work(self) -> bool:
        return bool(self.waiting_queue or self.prefilling_seqs or self.running_seqs)

    def get_stats(self) -> Dict[str, int]:
        return {"waiting": len(self.waiting_queue), "prefilling": len(self.prefilling_seqs),
                "running": len(self.running_seqs), "free_slots": len(self.free_slots)}

    # -- scheduling (scheduler_core.py:250-299) ---------------------------------

    def _schedule(self):
        admitted = []
        while self.waiting_queue and self.free_slots:
            seq = self.waiting_queue.popleft()
            slot = self.free_slots.popleft()
            seq.slot_id = slot
            seq.status = SeqStatus.PREFILLING
            self.slots[slot] = seq
            self.prefilling_seqs.append(seq)
            admitted.append(slot)
        if admitted:
            self.state_pool.zero_(torch.tensor(admitted, dtype=torch.long, device=self.device))
        decode_batch = list(self.running_seqs)[:self.max_batch_size]
        prefill_batch = []
        budget = self.max_batch_tokens
        for seq in list(self.prefilling_seqs):
            if budget <= 0:
                break
            n = min(len(seq.prompt_tokens) - seq.prefill_offset, self.prefill_chunk_size, budget)
            if n > 0:
                prefill_batch.append((seq, seq.prompt_tokens[seq.prefill_offset:seq.prefill_offset + n]))
                budget -= n
        return decode_batch, prefill_batch

    def _finish_sequence(self, seq: SequenceState) -> None:
        seq.status = SeqStatus.FINISHED
        if seq in self.running_seqs:
            self.running_seqs.remove(seq)
        if seq in self.prefilling_seqs:
            self.prefilling_seqs.remove(seq)
        self.slots[seq.slot_id] = None
        self.free_slots.append(seq.slot_id)

    # -- execution --------------------------------------------------------------

    def _i32(self, x):
        return torch.tensor(x, dtype=torch.int32).to(self.device, non_blocking=True)

    def _sample(self, logits: torch.Tensor, seqs: List[SequenceState]) -> List[Tuple[int, float]]:
        """One token per row with each sequence's own sampling settings
        (``TokenSampler.sample`` rules, ``scheduler_core.py:470-476, 563-569``)."""
        n = len(seqs)
        dev = self.device
        buf = SamplerBuffers(n, dev)
        buf.temperature.copy_(torch.tensor([float(s.temperature) for s in seqs], dtype=torch.float32))
        buf.top_p.copy_(torch.tensor([float(s.top_p) for s in seqs], dtype=torch.float32))
        buf.top_k.copy_(torch.tensor([int(s.top_k) for s in seqs], dtype=torch.int32))
        buf.rng_key.copy_(torch.tensor([s._rng_key for s in seqs], dtype=torch.int64))
        buf.rng_ctr.copy_(torch.tensor([len(s.generated_tokens) for s in seqs], dtype=torch.int32))
        if any(s.logit_bias for s in seqs):
            off, ids, vals = [0], [], []
            for s in seqs:
                for k, v in (s.logit_bias or {}).items():
                    ids.append(int(k))
                    vals.append(float(v))
                off.append(len(ids))
            buf.bias_off = self._i32(off)
            buf.bias_ids = self._i32(ids)
            buf.bias_val = torch.tensor(vals, dtype=torch.float32).to(dev)
        tok = torch.empty(n, dtype=torch.int64, device=dev)
        lp = torch.empty(n, dtype=torch.float32, device=dev)
        sample_rows(logits, buf, rule=RULE_SINGLE, max_valid_id=TokenSampler._max_valid_token_id,
                    seed=self._seed, out_tok=tok, out_logp=lp)
        return list(zip(tok.tolist(), lp.tolist()))

    def _append(self, seq: SequenceState, tok: int, lp: float, out: list) -> None:
        seq.last_token_id = tok
        seq.generated_tokens.append(tok)
        seq.generated_logps.append(lp)
        out.append((seq.seq_id, tok))
        if seq.is_finished:
            self._finish_sequence(seq)

    def _execute_decode(self, batch: List[SequenceState]) -> List[Tuple[Union[int, str], int]]:
        if not batch:
            return []
        if self.use_graph and not any(s.logit_bias for s in batch):
            # one graph replay; the step's one host synchronisation is the read of its tokens
            gr = self._graphs
            R = len(batch)
            Mb = gr.load(batch)
            gr.run(self._hip, self.state_pool, Mb, self._seed, TokenSampler._max_valid_token_id)
            toks, lps = gr.out_tok[:R].tolist(), gr.out_lp[:R].tolist()
            out = []
            for seq, t, lp in zip(batch, toks, lps):
                self._append(seq, t, lp, out)
            return out
        R = len(batch)
        tokens = torch.tensor([s.last_token_id for s in batch], dtype=torch.int64).to(self.device)
        rows = torch.arange(R, dtype=torch.int32, device=self.device)
        logits = self._hip.forward_pooled(tokens, self._i32([s.slot_id for s in batch]), rows, self.state_pool,
                                          decode=True)
        out = []
        for seq, (t, lp) in zip(batch, self._sample(logits, batch)):
            self._append(seq, t, lp, out)
        return out

    def _execute_prefill(self, batch) -> List[Tuple[Union[int, str], int]]:
        if not batch:
            return []
        toks, row_slot, row_last, cu, seq_slot, last_rows, done = [], [], [], [0], [], [], []
        for seq, chunk in batch:
            base = cu[-1]
            n = len(chunk)
            toks.extend(chunk)
            row_slot.extend([seq.slot_id] * n)
            row_last.extend([base + n - 1] + [-1] * (n - 1))
            cu.append(base + n)
            seq_slot.append(seq.slot_id)
            if seq.prefill_offset + n >= len(seq.prompt_tokens):
                last_rows.append(base + n - 1)
                done.append(seq)
        tokens = torch.tensor(toks, dtype=torch.int64).to(self.device)
        logits = self._hip.forward_pooled(tokens, self._i32(row_slot), self._i32(row_last), self.state_pool,
                                          decode=False, cu_seqlens=self._i32(cu), seq_slot=self._i32(seq_slot),
                                          logit_rows=self._i32(last_rows), n_logit_rows=len(last_rows))
        for seq, chunk in batch:
            seq.prefill_offset += len(chunk)
        out = []
        if done:
            picks = self._sample(logits, done)
            for seq, (t, lp) in zip(done, picks):
                seq.status = SeqStatus.RUNNING
                self.prefilling_seqs.remove(seq)
                self.running_seqs.append(seq)
                self._append(seq, t, lp, out)
        return out

    def step_sync(self) -> List[Tuple[Union[int, str], int]]:
        """One scheduling step: admit, decode the running sequences, prefill the
        next chunks; returns the step's new ``(seq_id, token_id)`` pairs."""
        with torch.no_grad():
            # re-bind the wrapper if the caller replaced parameters since the last step
            self._hip = as_hip_model(self.model)
            decode_batch, prefill_batch = self._schedule()
            if not decode_batch and not prefill_batch:
                return []
            new_tokens = self._execute_decode(decode_batch)
            new_tokens.extend(self._execute_prefill(prefill_batch))
            self._step_counter += 1
            return new_tokens

    def run_to_completion_sync(self) -> Iterator[List[Tuple[Union[int, str], int]]]:
        while self.has_pending_work():
            new = self.step_sync()
            if new:
                yield new

    async def step_async(self):
        return self.step_sync()


def create_scheduler_core(model, tokenizer, max_batch_size: int = 64, max_batch_tokens: int = 8192,
                          prefill_chunk_size: int = 512, state_cache=None) -> SchedulerCore:
    return SchedulerCore(model=model, tokenizer=tokenizer, max_batch_size=max_batch_size,
                         max_batch_tokens=max_batch_tokens, prefill_chunk_size=prefill_chunk_size,
                         state_cache=state_cache)
