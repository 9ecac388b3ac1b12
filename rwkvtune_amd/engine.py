"""Device-resident rollout engine: ragged prefill, fork-on-admit into a slot
pool, and a decode loop whose slot bookkeeping never leaves the GPU.

Used by the drop-in front ends (``GRPOBatchGenerator``, ``SchedulerCore``,
``BatchGenerator``).  One ``run`` is:

1. **Prefill** every distinct prompt once (ragged, packed, no padding and no
   length grouping) into a *prompt store* - a ``StatePool`` with one entry per
   distinct prompt - in passes of at most ``chunk_size`` tokens per prompt and
   ``max_batch_tokens`` tokens per forward.  The logits of each prompt's last
   token are kept.  (The reference prefills per exact-length group,
   ``grpo_batch_generator.py:353-431``, and the scheduler per slot,
   ``scheduler_core.py:513-600``.)
2. **First token** of every sequence from its prompt's logits, all sequences in
   one sampler launch (``grpo_batch_generator.py:262-310``).
3. **Decode**: ``n_slots`` slots hold live sequences.  A step is the model's
   fused single-token forward over the live rows, the sampler, and the commit
   kernel that appends tokens, retires finished sequences (EOS or per-sequence
   length), admits waiting ones into the freed slots by copying their prompt's
   state from the store (fork-on-admit: G generations of one prompt share one
   prefill) and packs the live slots into the leading rows.  A step runs the
   smallest row bucket (8, 16, multiples of 32 up to 256, then of 64 and 128)
   that covers the live rows, so the projections, row kernels and head shrink
   as the rollout drains; the host bounds the live rows by the sequences not
   yet known to be finished.  Below 32 rows every kernel runs the plan of 32
   rows (in the projections the tile's rows past the bucket read a zero page),
   so the 8- and 16-row steps give the 32-row step's results for their rows.
   Each bucket's step is captured once in a HIP graph and replayed; the graphs
   and every buffer they reference live in a decode context that is reused by
   later runs of the same configuration.  The host polls the
   finished-sequence counter every ``poll_every`` (2) steps through an
   asynchronous copy and reads the copy made one period earlier, so steps run
   back to back (2-4 steps stay queued) and at most 2 periods of all-idle
   steps follow the last finished sequence.
4. **Collect**: one copy of the token table back to the host.

Every sequence's tokens depend only on its prompt state, the logits of its
rows and its own (sequence, position) random stream, so results do not depend
on slot assignment or polling cadence.  Float32 models give the same tokens for
any slot count.  For 16-bit models the decode projections' plan (tile and K
split of the packed-weight GEMM; the head's own kernel and its row tile up to
128 rows, a library GEMM above) is chosen by
the step's row bucket, so float32 summation order, and with it a sampled token
now and then, can differ between runs with different slot counts; runs of one
configuration are bit-identical.
"""

from __future__ import annotations

import time
from typing import Dict, List, Optional, Sequence

import torch

from . import _lib
from .model import RWKV7Model, StatePool
from .sampler import RULE_BATCH, RULE_SINGLE, SamplerBuffers, repetition_penalty_, sample_rows

C_NEXT, C_DONE, C_STEP, C_NADMIT, C_LIVE = 0, 1, 2, 3, 4

ROW_BUCKETS = (8, 16, 32, 64, 96, 128, 160, 192, 224, 256, 320, 384, 448, 512, 640, 768, 896, 1024)


def row_buckets(S: int):
    """Row counts a decode step may run with ``S`` slots: the buckets below S, and S."""
    return sorted({b for b in ROW_BUCKETS if b < S} | {S})


def seq_keys(seed: int, n: int) -> torch.Tensor:
    """Per-sequence random-stream keys of a run (int64): distinct per (seed, sequence)."""
    base = (int(seed) * 0x9E3779B97F4A7C15) & 0x3FFFFFFFFFFFFFFF
    q = torch.arange(n, dtype=torch.int64)
    return (q * 0x2545F4914F6CDD1D + base) & 0x3FFFFFFFFFFFFFFF


class RolloutResult:
    """A run's output: ``ngen[q]`` tokens of sequence q in row q of the host
    tensors ``tok`` (int32), ``logp`` (float32) and ``step`` (int32, the decode
    step that produced each token, 0 = prefill), each ``[n, maxlen]``.  The
    per-sequence lists ``tokens``, ``logps`` and ``steps`` are built on first
    use, so a caller that needs only the ids pays for no Python lists."""

    def __init__(self, ngen: Sequence[int], tok: Optional[torch.Tensor], logp: Optional[torch.Tensor],
                 step: Optional[torch.Tensor], n_decode_steps: int, timings: Optional[Dict[str, float]] = None,
                 prompt_tokens: int = 0):
        self.ngen = [int(g) for g in ngen]
        self.tok, self.logp, self.step = tok, logp, step
        self.n_decode_steps = n_decode_steps
        self.timings = {} if timings is None else timings
        self.prompt_tokens = prompt_tokens
        self._lists = {}

    def _rows(self, name: str, t: Optional[torch.Tensor]) -> list:
        if name not in self._lists:
            self._lists[name] = [t[q, :g].tolist() for q, g in enumerate(self.ngen)] if t is not None else []
        return self._lists[name]

    @property
    def tokens(self) -> List[List[int]]:
        """Generated ids per sequence."""
        return self._rows("tokens", self.tok)

    @property
    def logps(self) -> List[List[float]]:
        """Sampling log-probabilities per token."""
        return self._rows("logps", self.logp)

    @property
    def steps(self) -> List[List[int]]:
        """Decode step that produced each token (0 = prefill)."""
        return self._rows("steps", self.step)

    def padded_ids(self):
        """(ids, mask): int64 ``[n, L]`` ids, zero past each sequence's end, and the
        bool mask of the generated positions, L = the longest sequence (1 when
        nothing was generated)."""
        n, L = len(self.ngen), max(self.ngen, default=0)
        if L == 0 or self.tok is None:
            ids = torch.zeros((n, 1), dtype=torch.long)
            return ids, torch.zeros_like(ids, dtype=torch.bool)
        mask = torch.arange(L)[None, :] < torch.tensor(self.ngen)[:, None]
        return self.tok[:, :L].long().masked_fill_(~mask, 0), mask


def _i32(x, dev):
    return torch.as_tensor(x, dtype=torch.int32).to(dev)


class RolloutEngine:
    """Slot-pool rollout on one GPU for a ``RWKV7Model``."""

    def __init__(self, model: RWKV7Model, n_slots: int, *, eos_token_id: Optional[int] = None,
                 max_valid_id: Optional[int] = None, use_graph: bool = True, poll_every: int = 2):
        if n_slots < 1 or n_slots > 1024:
            raise ValueError("n_slots must be in [1, 1024]")
        self.model = model
        self.n_slots = n_slots
        self.eos = -1 if eos_token_id is None else int(eos_token_id)
        self.max_valid_id = max_valid_id
        self.use_graph = use_graph
        self.poll_every = max(1, int(poll_every))
        self.dev = model.device
        self.pool = None

    def release(self):
        """Drop the cached decode context (prompt store, slot pool, sequence
        tables, captured graphs and their memory pool); the next ``run`` builds
        a new one.  Between rollouts the context holds
        ``(n_slots + distinct prompts) x`` a slot's state (1.5B: 13 MB, 7.2B:
        34 MB per slot) plus the token tables."""
        self._ctx = None

    # -- prefill ---------------------------------------------------------------

    def prefill_store(self, prompts: Sequence[Sequence[int]], chunk_size: int, max_batch_tokens: int,
                      max_seqs_per_forward: int = 0, store: Optional[StatePool] = None):
        """Prefill ``prompts`` into ``store`` (zeroed first; a new one when None);
        returns (store, last-token logits [U, V] float32)."""
        m = self.model
        dev = self.dev
        U = len(prompts)
        if store is None:
            store = StatePool(m.config, U, dev)
        else:
            store.zero_()
        V = m.config.vocab_size
        last_logits = torch.empty((U, V), dtype=torch.float32, device=dev)
        lens = [len(p) for p in prompts]
        if any(L == 0 for L in lens):
            raise ValueError("empty prompts are not supported")
        chunk = max(1, int(chunk_size))
        budget = max(1, int(max_batch_tokens))
        off = [0] * U
        while True:
            pending = [u for u in range(U) if off[u] < lens[u]]
            if not pending:
                break
            # one pass: every pending prompt advances by up to `chunk` tokens,
            # split into forwards of at most `budget` tokens
            group, gtok = [], 0
            groups = []
            for u in pending:
                n = min(chunk, lens[u] - off[u], budget)
                if group and (gtok + n > budget or 0 < max_seqs_per_forward <= len(group)):
                    groups.append(group)
                    group, gtok = [], 0
                group.append((u, n))
                gtok += n
            if group:
                groups.append(group)
            for grp in groups:
                self._prefill_group(prompts, grp, off, lens, store, last_logits)
            for grp in groups:
                for u, n in grp:
                    off[u] += n
        return store, last_logits

    def _prefill_group(self, prompts, grp, off, lens, store, last_logits):
        dev = self.dev
        toks, row_slot, row_last, cu, seq_slot, logit_rows, logit_dst = [], [], [], [0], [], [], []
        for u, n in grp:
            base = cu[-1]
            toks.extend(prompts[u][off[u]:off[u] + n])
            row_slot.extend([u] * n)
            row_last.extend([base + n - 1] + [-1] * (n - 1))
            cu.append(base + n)
            seq_slot.append(u)
            if off[u] + n == lens[u]:
                logit_rows.append(base + n - 1)
                logit_dst.append(u)
        tokens = torch.tensor(toks, dtype=torch.int64).to(dev, non_blocking=True)
        out = self.model.forward_pooled(tokens, _i32(row_slot, dev), _i32(row_last, dev), store, decode=False,
                                        cu_seqlens=_i32(cu, dev), seq_slot=_i32(seq_slot, dev),
                                        logit_rows=_i32(logit_rows, dev), n_logit_rows=len(logit_rows))
        if logit_rows:
            last_logits[torch.tensor(logit_dst, device=dev)] = out.float()

    # -- full rollout ------------------------------------------------------------

    def _context(self, key, n, maxlen, U, bias):
        """The decode context of this configuration: reused (with its captured
        graphs) when the key matches the previous run's, else built anew."""
        ctx = getattr(self, "_ctx", None)
        if ctx is not None and ctx.key == key and key is not None:
            return ctx
        self._ctx = None
        ctx = _DecodeCtx(key, self.model, self.n_slots, n, maxlen, U, bias, self.dev)
        self._ctx = ctx
        return ctx

    def _commit(self, c, have_sample: bool, n: int, maxlen: int, U: int):
        """The slot table's commit (append the step's samples, retire, admit into
        free slots, pack the live rows) and the admissions' state copies."""
        P = _lib.ptr
        cfg = self.model.config
        st = _lib.stream_of(c.counters)  # the stream current at call time (graph capture changes it)
        S = self.n_slots
        pool = c.pool
        _lib.call("rwkv7_rollout_commit", S, n, maxlen, int(have_sample), P(c.s_tok), P(c.s_lp),
                  P(c.slot_seq), P(c.row_slot), P(c.slot_row), P(c.tok_in), P(c.sp), P(c.seq_max_new),
                  P(c.seq_ngen), P(c.seq_done), P(c.out_tok), P(c.out_lp), P(c.out_step), self.eos,
                  P(c.counters), P(c.admit_slot), P(c.admit_src), st)
        _lib.call("rwkv7_admit_copy", P(c.counters), P(c.admit_slot), P(c.admit_src), cfg.n_layer, S, U,
                  cfg.n_head * 64 * 64, cfg.n_embd, P(c.store.kv), P(c.store.att_x), P(c.store.ffn_x),
                  P(pool.kv), P(pool.att_x), P(pool.ffn_x), st)

    def _step_body(self, c, Mb: int, n: int, maxlen: int, U: int, decode_rule: int, pen, per_seq):
        """One decode step over the leading ``Mb`` rows: the model's fused
        single-token forward, the sampler's per-row inputs, (the repetition
        penalty), the sampler, the commit."""
        P = _lib.ptr
        m = self.model
        S = self.n_slots
        logits = m.forward_pooled(c.tok_in[:Mb], c.row_slot[:Mb], c.row_last[:Mb], c.pool, decode=True)
        st = _lib.stream_of(c.counters)
        buf = c.buf
        s_temp, s_topp, s_topk = per_seq
        if pen is not None:
            penalty, flat, p_start, p_len, h_start, h_len, h2_start, h2_len = pen
            _lib.call("rwkv7_rollout_prepare", S, maxlen, P(c.row_slot), P(c.slot_seq), P(c.seq_key),
                      P(c.seq_ngen), P(c.sp), P(p_start), P(p_len), P(c.active), P(buf.rng_key),
                      P(buf.rng_ctr), P(h_start), P(h_len), P(h2_start), P(h2_len), P(s_temp), P(s_topp),
                      P(s_topk), P(buf.temperature), P(buf.top_p), P(buf.top_k), st)
            logits = logits.float()
            repetition_penalty_(logits, penalty, flat, h_start, h_len, c.out_tok.view(-1),
                                h2_start, h2_len, c.active)
        else:
            _lib.call("rwkv7_rollout_prepare", S, maxlen, P(c.row_slot), P(c.slot_seq), P(c.seq_key),
                      P(c.seq_ngen), None, None, None, P(c.active), P(buf.rng_key), P(buf.rng_ctr), None, None,
                      None, None, P(s_temp), P(s_topp), P(s_topk), P(buf.temperature), P(buf.top_p),
                      P(buf.top_k), st)
        sample_rows(logits, buf, rule=decode_rule, max_valid_id=self.max_valid_id, seed=0,
                    out_tok=c.s_tok, out_logp=c.s_lp, active=c.active)
        self._commit(c, True, n, maxlen, U)

    def _decode_step(self, c, bound: int, buckets, n: int, maxlen: int, U: int, decode_rule: int, pen, per_seq):
        """Run one decode step on the smallest row bucket covering ``bound`` live
        rows: the bucket's captured graph, captured on its second use (the first
        runs eagerly, so lazy allocations happen outside capture)."""
        ws = RWKV7Model.gemm_workspace(self.dev)
        if ws.ws.data_ptr() != c.ws_ptr:
            # the split-K workspace was reallocated: the captured graphs hold the old one
            c.graphs.clear()
            c.ws_ptr = ws.ws.data_ptr()
        Mb = next(b for b in buckets if b >= bound)
        g = c.graphs.get(Mb)
        if g is None and self.use_graph and Mb in c.warm:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=c.graph_pool):
                self._step_body(c, Mb, n, maxlen, U, decode_rule, pen, per_seq)
            c.graphs[Mb] = g
        if g is not None:
            g.replay()
        else:
            self._step_body(c, Mb, n, maxlen, U, decode_rule, pen, per_seq)
            c.warm.add(Mb)

    @torch.no_grad()
    def run(self, prompts: Sequence[Sequence[int]], seq_prompt: Sequence[int], max_new_tokens,
            *, temperature: float = 1.0, top_p: float = 1.0, top_k: int = 0, logit_bias: Optional[dict] = None,
            repetition_penalty: float = 1.0, first_rule: int = RULE_SINGLE, decode_rule: int = RULE_BATCH,
            first_can_finish: bool = True, chunk_size: int = 2048, max_batch_tokens: int = 1 << 20,
            seed: int = 0, max_len_cap: Optional[int] = None, per_seq_sampling=None,
            max_seqs_per_forward: int = 0) -> RolloutResult:
        """Roll out ``len(seq_prompt)`` sequences; sequence q continues prompt
        ``prompts[seq_prompt[q]]``.  ``per_seq_sampling``: optional
        ``(temperature[n], top_p[n], top_k[n])`` overriding the scalars per sequence."""
        m = self.model
        dev = self.dev
        n = len(seq_prompt)
        S = self.n_slots
        if isinstance(max_new_tokens, int):
            max_new = [int(max_new_tokens)] * n
        else:
            max_new = [int(x) for x in max_new_tokens]
        if n == 0:
            return RolloutResult([], None, None, None, 0)
        if min(max_new) < 1:
            raise ValueError("max_new_tokens must be >= 1")
        # a sequence whose first token cannot finish it makes at least one decode step
        maxlen = max(max(max_new), 1 if first_can_finish else 2)
        if max_len_cap is not None:
            maxlen = min(maxlen, max_len_cap)
        U = len(prompts)
        use_pen = repetition_penalty != 1.0 and repetition_penalty > 0
        bias = tuple(sorted((int(k), float(v)) for k, v in (logit_bias or {}).items()))
        # what the captured step graphs bake in; runs with the repetition penalty
        # (prompt-sized tables) or per-sequence sampling are not cached
        m.packs()
        ws = RWKV7Model.gemm_workspace(dev)
        key = None if (use_pen or per_seq_sampling is not None) else (
            S, n, maxlen, U, self.eos, decode_rule, self.max_valid_id, bias, m._packs_gen, ws.ws.data_ptr())
        timings = {}
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        ctx = self._context(key, n, maxlen, U, bias)

        # 1. prefill distinct prompts into the context's store
        _, last_logits = self.prefill_store(prompts, chunk_size, max_batch_tokens, max_seqs_per_forward,
                                            store=ctx.store)
        torch.cuda.synchronize(dev)
        t1 = time.perf_counter()
        timings["prefill_s"] = t1 - t0

        # sequence table of this run
        ctx.reset(seq_prompt, max_new, seq_keys(seed, n), temperature, top_p, top_k)
        plen = [len(p) for p in prompts]
        if use_pen:
            pstart = [0]
            for L in plen[:-1]:
                pstart.append(pstart[-1] + L)
            flat = torch.tensor([t for p in prompts for t in p], dtype=torch.int32).to(dev)
            p_start = torch.tensor(pstart, dtype=torch.int64).to(dev)
            p_len = _i32(plen, dev)
            h_start = torch.zeros(S, dtype=torch.int64, device=dev)
            h_len = torch.zeros(S, dtype=torch.int32, device=dev)
            h2_start = torch.zeros(S, dtype=torch.int64, device=dev)
            h2_len = torch.zeros(S, dtype=torch.int32, device=dev)
        if per_seq_sampling is not None:
            s_temp = torch.tensor(per_seq_sampling[0], dtype=torch.float32).to(dev)
            s_topp = torch.tensor(per_seq_sampling[1], dtype=torch.float32).to(dev)
            s_topk = torch.tensor(per_seq_sampling[2], dtype=torch.int32).to(dev)
        else:
            s_temp = s_topp = s_topk = None

        # 2. first token of every sequence
        P = _lib.ptr
        c = ctx
        cur = lambda: _lib.stream_of(c.counters)  # the stream current at call time (graph capture changes it)
        fbuf = SamplerBuffers(n, dev)
        fbuf.set_uniform(temperature, top_p, top_k)
        if per_seq_sampling is not None:
            fbuf.temperature.copy_(s_temp)
            fbuf.top_p.copy_(s_topp)
            fbuf.top_k.copy_(s_topk)
        fbuf.set_bias(logit_bias, n)
        fbuf.rng_key.copy_(c.seq_key)
        fbuf.rng_ctr.zero_()
        f_tok = torch.empty(n, dtype=torch.int64, device=dev)
        f_lp = torch.empty(n, dtype=torch.float32, device=dev)
        CH = 1024
        for a in range(0, n, CH):
            b = min(n, a + CH)
            lg = last_logits.index_select(0, c.sp[a:b].long())
            if use_pen:
                idx = c.sp[a:b].long()
                repetition_penalty_(lg, repetition_penalty, flat, p_start[idx], p_len[idx])
            sub = SamplerBuffers.__new__(SamplerBuffers)
            sub.temperature, sub.top_p, sub.top_k = fbuf.temperature[a:b], fbuf.top_p[a:b], fbuf.top_k[a:b]
            sub.rng_key, sub.rng_ctr = fbuf.rng_key[a:b], fbuf.rng_ctr[a:b]
            sub.bias_off = fbuf.bias_off[: b - a + 1] if fbuf.bias_off is not None else None
            sub.bias_ids, sub.bias_val = fbuf.bias_ids, fbuf.bias_val
            sample_rows(lg, sub, rule=first_rule, max_valid_id=self.max_valid_id, seed=0,
                        out_tok=f_tok[a:b], out_logp=f_lp[a:b])
        _lib.call("rwkv7_rollout_first", n, maxlen, P(f_tok), P(f_lp), P(c.seq_max_new), P(c.seq_ngen),
                  P(c.seq_done), P(c.out_tok), P(c.out_lp), P(c.out_step), self.eos, int(first_can_finish),
                  P(c.counters), cur())
        del last_logits

        # 3. decode
        pen = (repetition_penalty, flat, p_start, p_len, h_start, h_len, h2_start, h2_len) if use_pen else None
        per_seq = (s_temp, s_topp, s_topk)
        self._commit(c, False, n, maxlen, U)  # initial admission
        torch.cuda.synchronize(dev)
        t2 = time.perf_counter()
        timings["first_token_s"] = t2 - t1

        buckets = row_buckets(S)
        h_done = torch.zeros(2, dtype=torch.int32).pin_memory()
        cap = n * maxlen + 16
        n_steps = 0
        pending_evt = None
        done = False
        finished = 0  # sequences known to be finished (from the last completed poll)
        while not done and n_steps < cap:
            for _ in range(self.poll_every):
                # rows needed: the live rows are at most the sequences not known to be finished
                self._decode_step(c, min(S, n - finished), buckets, n, maxlen, U, decode_rule, pen, per_seq)
                n_steps += 1
            # read the counters copied one polling period ago (already complete
            # unless the GPU is behind), then queue a fresh copy
            if pending_evt is not None:
                pending_evt.synchronize()
                finished = int(h_done[0])
                if finished >= n:
                    done = True
            h_done[0:2].copy_(c.counters[1:3], non_blocking=True)
            pending_evt = torch.cuda.Event()
            pending_evt.record()
        torch.cuda.synchronize(dev)
        if int(h_done[0]) < n:
            h = c.counters.cpu()
            if int(h[C_DONE]) < n:
                raise RuntimeError(f"rollout did not finish: {int(h[C_DONE])}/{n} sequences after {n_steps} steps")
        t3 = time.perf_counter()
        timings["decode_s"] = t3 - t2

        # 4. collect: host copies of the output tables (the context's buffers are
        # reused by the next run); the per-sequence lists are built on demand
        ng = c.seq_ngen.cpu().tolist()
        ot = c.out_tok.cpu()
        ol = c.out_lp.cpu()
        os_ = c.out_step.cpu()
        n_dec = int(c.counters[C_STEP].item())
        t4 = time.perf_counter()
        timings["collect_s"] = t4 - t3
        timings["total_s"] = t4 - t0
        timings["decode_steps_issued"] = n_steps
        if key is None:
            self._ctx = None  # uncached: drop its buffers and graphs
        return RolloutResult(ng, ot, ol, os_, n_dec, timings, prompt_tokens=sum(plen))


    @torch.no_grad()
    def run_inline(self, prompts: Sequence[Sequence[int]], max_new_tokens, *, temperature: float = 1.0,
                   top_p: float = 1.0, top_k: int = 0, logit_bias: Optional[dict] = None,
                   first_rule: int = RULE_SINGLE, decode_rule: int = RULE_SINGLE, chunk_size: int = 512,
                   max_batch_tokens: int = 8192, seed: int = 0, per_seq_sampling=None) -> RolloutResult:
        """Continuous batching with every prompt prefilled in its own slot, for
        queues longer than the slot pool (``SchedulerCore`` semantics,
        ``rwkvtune/inference/scheduler_core.py:250-299, 445-600``): sequence q
        continues ``prompts[q]``; its first token may finish it.

        * The decode step's commit kernel admits waiting sequences (index order)
          into freed slots on the device and zeroes their state; an admitted
          sequence holds no row until it has a token.
        * The host learns of admissions from its asynchronous poll (no step waits
          for it) and prefills the admitted prompts straight into their slots,
          ``chunk_size`` tokens per sequence and at most ``max_batch_tokens`` per
          forward, one ragged forward between polling periods of decode steps.
        * When a prompt is complete, its first token is drawn from the prompt's
          last logits and recorded on the device (``rwkv7_rollout_activate``); the
          next commit gives the slot a row, or frees it if that token finished
          the sequence.
        Memory is the slot pool and the token tables, whatever the queue length.
        Tokens depend only on each sequence's prompt and (sequence, position)
        random stream, as in ``run``."""
        m = self.model
        dev = self.dev
        n = len(prompts)
        S = self.n_slots
        if isinstance(max_new_tokens, int):
            max_new = [int(max_new_tokens)] * n
        else:
            max_new = [int(x) for x in max_new_tokens]
        if n == 0:
            return RolloutResult([], None, None, None, 0)
        if min(max_new) < 1:
            raise ValueError("max_new_tokens must be >= 1")
        lens = [len(p) for p in prompts]
        if min(lens) < 1:
            raise ValueError("empty prompts are not supported")
        maxlen = max(max_new)
        chunk = max(1, int(chunk_size))
        budget = max(1, int(max_batch_tokens))
        bias = tuple(sorted((int(k), float(v)) for k, v in (logit_bias or {}).items()))
        m.packs()
        ws = RWKV7Model.gemm_workspace(dev)
        # one zero store entry: admission zeroes the slot (the prompt is prefilled there)
        key = None if per_seq_sampling is not None else (
            "inline", S, n, maxlen, self.eos, decode_rule, self.max_valid_id, bias, m._packs_gen, ws.ws.data_ptr())
        timings = {}
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        c = self._context(key, n, maxlen, 1, bias)
        c.reset([0] * n, max_new, seq_keys(seed, n), temperature, top_p, top_k)
        if per_seq_sampling is not None:
            s_temp = torch.tensor(per_seq_sampling[0], dtype=torch.float32).to(dev)
            s_topp = torch.tensor(per_seq_sampling[1], dtype=torch.float32).to(dev)
            s_topk = torch.tensor(per_seq_sampling[2], dtype=torch.int32).to(dev)
        else:
            s_temp = s_topp = s_topk = None
        per_seq = (s_temp, s_topp, s_topk)
        # first-token sampler inputs for up to S sequences at a time (bias tables built once)
        fbuf = SamplerBuffers(S, dev)
        fbuf.set_uniform(temperature, top_p, top_k)
        fbuf.set_bias(logit_bias, S)
        fbuf.rng_ctr.zero_()
        f_tok = torch.empty(S, dtype=torch.int64, device=dev)
        f_lp = torch.empty(S, dtype=torch.float32, device=dev)
        P = _lib.ptr
        st = lambda: _lib.stream_of(c.counters)

        # host view of the sequences: 0 not seen admitted, 1 prefilling, 2 first token recorded
        hstate = [0] * n
        slot_of = [-1] * n
        pf_off = [0] * n
        pend: List[int] = []
        activated = 0

        def take(snapshot):
            new = [(int(q), sl) for sl, q in enumerate(snapshot) if q >= 0 and hstate[int(q)] == 0]
            for q, sl in sorted(new):
                hstate[q] = 1
                slot_of[q] = sl
                pend.append(q)

        def pinned(vals, dtype):
            t = torch.tensor(vals, dtype=dtype).pin_memory()
            return t.to(dev, non_blocking=True)

        def prefill_pass():
            """One ragged forward over the next chunks of the prefilling prompts
            (admission order), then the first tokens of the completed ones."""
            nonlocal activated
            room = budget
            batch = []
            for q in pend:
                k = min(chunk, lens[q] - pf_off[q], room)
                if k <= 0:
                    break
                batch.append((q, k))
                room -= k
                if room <= 0:
                    break
            toks, row_slot, row_last, seq_slot, logit_rows, done_q = [], [], [], [], [], []
            cu = [0]
            for q, k in batch:
                base = cu[-1]
                toks.extend(prompts[q][pf_off[q]:pf_off[q] + k])
                row_slot.extend([slot_of[q]] * k)
                row_last.extend([base + k - 1] + [-1] * (k - 1))
                cu.append(base + k)
                seq_slot.append(slot_of[q])
                if pf_off[q] + k == lens[q]:
                    logit_rows.append(base + k - 1)
                    done_q.append(q)
            logits = m.forward_pooled(pinned(toks, torch.int64), pinned(row_slot, torch.int32),
                                      pinned(row_last, torch.int32), c.pool, decode=False,
                                      cu_seqlens=pinned(cu, torch.int32), seq_slot=pinned(seq_slot, torch.int32),
                                      logit_rows=pinned(logit_rows, torch.int32),
                                      n_logit_rows=len(done_q))
            for q, k in batch:
                pf_off[q] += k
            if not done_q:
                return
            for q in done_q:
                hstate[q] = 2
                pend.remove(q)
            k = len(done_q)
            idx = pinned(done_q, torch.int32)
            sub = SamplerBuffers.__new__(SamplerBuffers)
            if s_temp is not None:
                il = idx.long()
                sub.temperature, sub.top_p, sub.top_k = s_temp[il], s_topp[il], s_topk[il]
            else:
                sub.temperature, sub.top_p, sub.top_k = fbuf.temperature[:k], fbuf.top_p[:k], fbuf.top_k[:k]
            sub.rng_key = c.seq_key.index_select(0, idx.long())
            sub.rng_ctr = fbuf.rng_ctr[:k]
            sub.bias_off = fbuf.bias_off[: k + 1] if fbuf.bias_off is not None else None
            sub.bias_ids, sub.bias_val = fbuf.bias_ids, fbuf.bias_val
            sample_rows(logits, sub, rule=first_rule, max_valid_id=self.max_valid_id, seed=0,
                        out_tok=f_tok[:k], out_logp=f_lp[:k])
            _lib.call("rwkv7_rollout_activate", k, P(idx), n, maxlen, P(f_tok), P(f_lp), P(c.seq_max_new),
                      P(c.seq_ngen), P(c.seq_done), P(c.out_tok), P(c.out_lp), P(c.out_step), self.eos, 1,
                      P(c.counters), st())
            # rows for the new sequences; slots their first token finished are refilled
            self._commit(c, False, n, maxlen, 1)
            activated += k

        # initial admission (every slot free), read back once
        self._commit(c, False, n, maxlen, 1)
        take(c.slot_seq.cpu().tolist())
        buckets = row_buckets(S)
        snap = torch.zeros(3 + S, dtype=torch.int32).pin_memory()
        cap = n * maxlen + sum((L + chunk - 1) // chunk for L in lens) + 16
        n_steps = n_prefill = idle = 0
        pending_evt = None
        finished = 0
        t_prefill = 0.0
        while finished < n:
            progressed = False
            if pend:
                tp = time.perf_counter()
                prefill_pass()
                t_prefill += time.perf_counter() - tp
                n_prefill += 1
                progressed = True
            live_bound = min(S, activated - finished)
            if live_bound > 0:
                for _ in range(self.poll_every):
                    self._decode_step(c, live_bound, buckets, n, maxlen, 1, decode_rule, None, per_seq)
                    n_steps += 1
                progressed = True
            if pending_evt is not None:
                pending_evt.synchronize()
                finished = int(snap[1])
                take(snap[3:].tolist())
            snap[0:3].copy_(c.counters[0:3], non_blocking=True)
            snap[3:].copy_(c.slot_seq, non_blocking=True)
            pending_evt = torch.cuda.Event()
            pending_evt.record()
            idle = 0 if progressed else idle + 1
            if n_steps + n_prefill > cap or idle > 64:
                raise RuntimeError(f"rollout did not finish: {finished}/{n} sequences after {n_steps} decode "
                                   f"steps and {n_prefill} prefill passes")
        torch.cuda.synchronize(dev)
        t3 = time.perf_counter()
        timings["prefill_host_s"] = t_prefill
        timings["decode_s"] = t3 - t0
        timings["prefill_passes"] = n_prefill
        ng = c.seq_ngen.cpu().tolist()
        ot, ol, os_ = c.out_tok.cpu(), c.out_lp.cpu(), c.out_step.cpu()
        n_dec = int(c.counters[C_STEP].item())
        t4 = time.perf_counter()
        timings["collect_s"] = t4 - t3
        timings["total_s"] = t4 - t0
        timings["decode_steps_issued"] = n_steps
        if key is None:
            self._ctx = None
        return RolloutResult(ng, ot, ol, os_, n_dec, timings, prompt_tokens=sum(lens))


class _DecodeCtx:
    """Every buffer a decode step reads or writes, for one configuration (slots,
    sequences, token columns, prompts, logit bias): the prompt store, the slot
    pool, the sequence / slot / row tables, the sampler's per-row inputs and the
    captured step graph of each row bucket.  Kept by the engine so that later
    runs of the same configuration replay the same graphs."""

    def __init__(self, key, model, S, n, maxlen, U, bias, dev):
        self.key = key
        cfg = model.config
        self.store = StatePool(cfg, U, dev)
        self.pool = StatePool(cfg, S, dev)
        self.sp = torch.zeros(n, dtype=torch.int32, device=dev)
        self.seq_max_new = torch.zeros(n, dtype=torch.int32, device=dev)
        self.seq_key = torch.zeros(n, dtype=torch.int64, device=dev)
        self.seq_ngen = torch.zeros(n, dtype=torch.int32, device=dev)
        self.seq_done = torch.zeros(n, dtype=torch.uint8, device=dev)
        self.out_tok = torch.zeros((n, maxlen), dtype=torch.int32, device=dev)
        self.out_lp = torch.zeros((n, maxlen), dtype=torch.float32, device=dev)
        self.out_step = torch.zeros((n, maxlen), dtype=torch.int32, device=dev)
        self.counters = torch.zeros(8, dtype=torch.int32, device=dev)
        self.slot_seq = torch.full((S,), -1, dtype=torch.int32, device=dev)
        self.row_slot = torch.full((S,), -1, dtype=torch.int32, device=dev)
        self.slot_row = torch.full((S,), -1, dtype=torch.int32, device=dev)
        self.row_last = torch.arange(S, dtype=torch.int32, device=dev)
        self.tok_in = torch.zeros(S, dtype=torch.int64, device=dev)
        self.admit_slot = torch.zeros(S, dtype=torch.int32, device=dev)
        self.admit_src = torch.zeros(S, dtype=torch.int32, device=dev)
        self.s_tok = torch.zeros(S, dtype=torch.int64, device=dev)
        self.s_lp = torch.zeros(S, dtype=torch.float32, device=dev)
        self.active = torch.zeros(S, dtype=torch.uint8, device=dev)
        self.buf = SamplerBuffers(S, dev)
        self.buf.set_bias(dict(bias) if bias else None, S)
        self.graphs: Dict[int, torch.cuda.CUDAGraph] = {}
        self.warm = set()
        self.graph_pool = torch.cuda.graph_pool_handle()
        self.ws_ptr = RWKV7Model.gemm_workspace(dev).ws.data_ptr()

    def reset(self, seq_prompt, max_new, keys, temperature, top_p, top_k):
        self.sp.copy_(torch.as_tensor(seq_prompt, dtype=torch.int32))
        self.seq_max_new.copy_(torch.as_tensor(max_new, dtype=torch.int32))
        self.seq_key.copy_(keys)
        for t in (self.seq_ngen, self.seq_done, self.out_tok, self.out_lp, self.out_step, self.counters,
                  self.tok_in, self.s_tok, self.s_lp, self.active):
            t.zero_()
        for t in (self.slot_seq, self.row_slot, self.slot_row):
            t.fill_(-1)
        # (the slot pool needs no clearing: admission copies a slot's whole state)
        self.buf.set_uniform(temperature, top_p, top_k)
