"""GPU slot-table rollout (rwkvtune_amd.engine and its front ends) against the
CPU restatement of the reference loops (oracle/rollout.py).

Greedy decoding is deterministic, so token ids must be identical per sequence
(float32 model).  Sampled decoding is checked for invariance: the tokens of every
sequence depend only on its prompt and its (sequence, position) random stream,
so changing the slot count, the HIP-graph switch or the polling cadence must not
change a single token (the race detector for the slot table).
"""

import pytest
import torch

from oracle import model as om
from oracle import rollout as orl
from rwkvtune_amd.batch_generator import BatchGenerator, GenerationConfig
from rwkvtune_amd.engine import RolloutEngine, row_buckets
from rwkvtune_amd.grpo_batch_generator import GRPOBatchGenerator
from rwkvtune_amd.model import RWKV7Config, build_model
from rwkvtune_amd.sampler import RULE_BATCH, RULE_SINGLE, TokenSampler
from rwkvtune_amd.scheduler_core import SchedulerCore, SequenceState

pytestmark = pytest.mark.gpu

V = 1000


class TinyTok:
    """Stand-in tokenizer: ids 0..V-4 decodable, so the top 3 ids are banned."""
    eos_token_id = None

    def __init__(self, eos=None):
        self.idx2token = {i: str(i).encode() for i in range(V - 3)}
        self.eos_token_id = eos

    def decode(self, ids):
        return " ".join(str(i) for i in ids)

    def encode(self, s):
        return [int(x) for x in s.split()]


@pytest.fixture(scope="module")
def tiny(gpu_device):
    cfg = RWKV7Config(n_layer=2, n_embd=256, vocab_size=V, dim_att_lora=32, dim_gate_lora=64, dim_mv_lora=32)
    m = build_model(cfg, dtype=torch.float32, device="cuda", seed=21)
    sd = om.cast_state_dict(m.state_dict(), torch.float32)
    return m, sd


def prompts(seed, n, lo, hi):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (n,), generator=g).tolist()
    return [torch.randint(0, V - 3, (L,), generator=g).tolist() for L in lens]


def test_grpo_greedy_matches_reference_loop(tiny):
    print("[case] GRPO greedy parity", flush=True)
    m, sd = tiny
    ps = prompts(1, 4, 3, 40)
    ps.append(list(ps[1]))  # a duplicate prompt: prefilled once, forked
    G, max_new = 3, 12
    caps = [max_new - (i % 5) for i in range(len(ps) * G)]
    free, _ = orl.grpo_rollout(sd, ps, max_new, G, max_valid_id=V - 4, caps=caps)
    eos = free[0][3]  # a token greedy decoding produces, so the EOS path is exercised
    ref, _ = orl.grpo_rollout(sd, ps, max_new, G, eos=eos, max_valid_id=V - 4, caps=caps)
    gen = GRPOBatchGenerator(m, TinyTok(), chunk_size=16, max_decode_batch_size=4, eos_token_id=eos, verbose=False)
    out = gen.generate(ps, max_new, num_generations=G, temperature=0.0, top_p=1.0, max_new_tokens_per_seq=caps)
    ids, masks = out["completion_ids"].cpu(), out["masks"].cpu()
    assert ids.shape[0] == len(ps) * G and ids.dtype == torch.long and masks.dtype == torch.bool
    for q, r in enumerate(ref):
        n = int(masks[q].sum())
        assert ids[q, :n].tolist() == r, f"path {q}"
        assert bool((ids[q, n:] == 0).all())
        assert out["completions"][q] == " ".join(map(str, r))
    assert any(r[-1] == eos and len(r) < caps[q] for q, r in enumerate(ref)), "EOS path not exercised"


def test_scheduler_and_batch_generator_greedy(tiny):
    print("[case] SchedulerCore / BatchGenerator greedy parity", flush=True)
    m, sd = tiny
    ps = prompts(2, 6, 1, 30)
    free = orl.scheduler_rollout(sd, ps, 10, max_valid_id=V - 4)
    eos = free[2][4]
    ref = orl.scheduler_rollout(sd, ps, 10, eos=eos, max_valid_id=V - 4)
    sch = SchedulerCore(m, TinyTok(eos), max_batch_size=3, max_batch_tokens=50, prefill_chunk_size=7)
    seqs = [SequenceState(seq_id=i, prompt_tokens=p, max_new_tokens=10, temperature=0.0, eos_token_id=eos)
            for i, p in enumerate(ps)]
    sch.add_sequences(seqs)
    got = {i: [] for i in range(len(ps))}
    for upd in sch.run_to_completion_sync():
        for sid, t in upd:
            got[sid].append(t)
    assert not sch.has_pending_work()
    for i, r in enumerate(ref):
        assert got[i] == r and seqs[i].generated_tokens == r
    # BatchGenerator strips a trailing EOS and returns float masks
    bg = BatchGenerator(m, TinyTok(eos))
    res = bg.generate(input_ids=ps, generation_config=GenerationConfig(max_length=10, temperature=0.0,
                                                                      chunk_size=9, num_generations=2))
    assert res["masks"].dtype == torch.float32 and res["completion_ids"].shape[0] == 2 * len(ps)
    for i, r in enumerate(ref):
        exp = r[:-1] if r[-1] == eos else r
        for g in range(2):
            row = res["completion_ids"][2 * i + g].cpu()
            n = int(res["masks"][2 * i + g].sum())
            assert row[:n].tolist() == exp


@pytest.mark.parametrize("rule", [RULE_BATCH, RULE_SINGLE])
def test_sampled_rollout_invariant_to_slots_and_graphs(tiny, rule):
    print(f"[case] sampled rollout invariance rule={rule}", flush=True)
    m, _ = tiny
    ps = prompts(3, 5, 5, 60)
    seq_prompt = [i // 4 for i in range(20)]
    caps = [3 + (7 * i) % 17 for i in range(20)]
    kw = dict(temperature=1.0, top_p=0.95, top_k=0, first_rule=RULE_SINGLE, decode_rule=rule,
              first_can_finish=False, chunk_size=13, seed=1234)
    runs = []
    for slots, graph, poll in ((3, True, 2), (20, True, 8), (7, False, 1)):
        eng = RolloutEngine(m, slots, eos_token_id=None, max_valid_id=V - 4, use_graph=graph, poll_every=poll)
        res = eng.run(ps, seq_prompt, caps, **kw)
        runs.append(res)
        for q, t in enumerate(res.tokens):
            assert len(t) == caps[q]
            assert max(t) <= V - 4 and min(t) >= 0
            assert all(lp <= 1e-6 for lp in res.logps[q])
    for r in runs[1:]:
        assert r.tokens == runs[0].tokens


def test_repetition_penalty_greedy(tiny):
    """Greedy GRPO with a strong repetition penalty equals the reference loop
    with the penalty applied to prompt + generated ids."""
    print("[case] repetition penalty rollout", flush=True)
    m, sd = tiny
    ps = prompts(4, 3, 4, 20)
    pen = 3.0

    def ref_one(p, n):
        from oracle import sampler as osm
        lg, st = om.forward_with_state(sd, torch.tensor([p]), None, torch.float32)
        toks = []
        while len(toks) < n:
            row = osm.repetition_penalty(lg[0, -1:], [p + toks], pen)[0]
            toks.append(osm.greedy(row, V - 4)[0])
            lg, st = om.forward_with_state(sd, torch.tensor([[toks[-1]]]), st, torch.float32)
        return toks

    gen = GRPOBatchGenerator(m, TinyTok(), max_decode_batch_size=2, verbose=False)
    out = gen.generate(ps, 8, num_generations=1, temperature=0.0, repetition_penalty=pen)
    for i, p in enumerate(ps):
        assert out["completion_ids"][i].cpu().tolist() == ref_one(p, 8)


def _run_scheduler(m, tok, seqs, slots, budget=64, chunk=8):
    sch = SchedulerCore(m, tok, max_batch_size=slots, max_batch_tokens=budget, prefill_chunk_size=chunk)
    sch.add_sequences(seqs)
    steps = 0
    for _ in sch.run_to_completion_sync():
        steps += 1
    assert not sch.has_pending_work()
    return sch, steps


def test_scheduler_bounded_memory_long_queue(tiny):
    """2000 distinct prompts through 64 slots: the slot pool is the only state,
    so peak device memory does not grow with the queue (a state per prompt
    would add ~264 MB here); every sequence ends at its cap and greedy ids equal
    the per-sequence restatement of the reference loop (checked on every 40th)."""
    print("[case] SchedulerCore 2000 prompts / 64 slots", flush=True)
    m, sd = tiny
    tok = TinyTok()

    def peak_for(n, seed):
        ps = prompts(seed, n, 2, 6)
        seqs = [SequenceState(seq_id=i, prompt_tokens=p, max_new_tokens=3, temperature=0.0) for i, p in enumerate(ps)]
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        _run_scheduler(m, tok, seqs, 64)
        torch.cuda.synchronize()
        return ps, seqs, torch.cuda.max_memory_allocated() - base

    _, _, peak_small = peak_for(200, 40)
    ps, seqs, peak_big = peak_for(2000, 41)
    print(f"  peak extra memory: 200 prompts {peak_small / 2**20:.1f} MiB, 2000 prompts {peak_big / 2**20:.1f} MiB",
          flush=True)
    assert peak_big <= peak_small + (8 << 20)
    assert all(len(s.generated_tokens) == 3 and s.status.name == "FINISHED" for s in seqs)
    sub = list(range(0, 2000, 40))
    ref = orl.scheduler_rollout(sd, [ps[i] for i in sub], 3, max_valid_id=V - 4)
    for i, r in zip(sub, ref):
        assert seqs[i].generated_tokens == r, i


def test_scheduler_streams_and_admits_midrun(tiny):
    """step_sync hands out each step's tokens as they are made; sequences added
    after the run started are admitted into the running pool and finish too;
    every sequence equals the reference loop (greedy, EOS)."""
    print("[case] SchedulerCore streaming + mid-run admission", flush=True)
    m, sd = tiny
    ps = prompts(42, 10, 1, 25)
    free = orl.scheduler_rollout(sd, ps, 9, max_valid_id=V - 4)
    eos = free[1][3]
    ref = orl.scheduler_rollout(sd, ps, 9, eos=eos, max_valid_id=V - 4)
    sch = SchedulerCore(m, TinyTok(eos), max_batch_size=4, max_batch_tokens=20, prefill_chunk_size=6)
    seqs = [SequenceState(seq_id=i, prompt_tokens=p, max_new_tokens=9, temperature=0.0, eos_token_id=eos)
            for i, p in enumerate(ps)]
    sch.add_sequences(seqs[:5])
    got = {i: [] for i in range(10)}
    n_updates = 0
    for _ in range(4):
        for sid, t in sch.step_sync():
            got[sid].append(t)
            n_updates += 1
    assert sch.has_pending_work() and n_updates > 0
    sch.add_sequences(seqs[5:])
    for upd in sch.run_to_completion_sync():
        for sid, t in upd:
            got[sid].append(t)
    for i, r in enumerate(ref):
        assert got[i] == r and seqs[i].generated_tokens == r, i


def test_scheduler_sampled_streams_independent_of_slots(tiny):
    """Draws are keyed by (sequence, position): the sampled tokens of every
    sequence are the same with 2 and with 7 slots."""
    print("[case] SchedulerCore sampled invariance", flush=True)
    m, _ = tiny
    ps = prompts(43, 7, 2, 20)
    runs = []
    for slots in (2, 7):
        TokenSampler.manual_seed(1234)
        seqs = [SequenceState(seq_id=i, prompt_tokens=p, max_new_tokens=8, temperature=0.9, top_p=0.9,
                              top_k=40 if i % 2 else 0) for i, p in enumerate(ps)]
        _run_scheduler(m, TinyTok(), seqs, slots, budget=30, chunk=5)
        runs.append([s.generated_tokens for s in seqs])
    assert runs[0] == runs[1]
    assert all(len(t) == 8 for t in runs[0])


def test_row_buckets_greedy_parity_and_graph_reuse(tiny):
    """96 slots run rows in buckets of 8 / 16 / 32 / 64 / 96 as the rollout drains
    (live slots packed into the leading rows): 150 greedy paths with caps 1..24
    equal the reference loop, and the drain captured graphs of buckets below 32
    rows.  A second engine run of the same configuration replays
    the first run's captured graphs: a sampled run with a new seed equals the
    same seed's run on a fresh engine, and repeating a seed repeats the tokens."""
    print("[case] row buckets: parity across buckets, graph reuse", flush=True)
    m, sd = tiny
    ps = prompts(50, 50, 2, 12)
    g = torch.Generator().manual_seed(51)
    caps = torch.randint(1, 25, (150,), generator=g).tolist()
    gen = GRPOBatchGenerator(m, TinyTok(), chunk_size=16, max_decode_batch_size=96, verbose=False)
    out = gen.generate(ps, 24, num_generations=3, temperature=0.0, top_p=1.0, max_new_tokens_per_seq=caps)
    ref, _ = orl.grpo_rollout(sd, ps, 24, 3, max_valid_id=V - 4, caps=caps)
    ids, masks = out["completion_ids"].cpu(), out["masks"].cpu()
    for q, r in enumerate(ref):
        assert ids[q, :int(masks[q].sum())].tolist() == r, q
    eng = gen._engines[96]
    got = set(eng._ctx.graphs)
    assert {64, 96} <= got <= set(row_buckets(96)) and min(got) < 32, sorted(got)

    def sampled(generator, seed):
        o = generator.generate(ps, 24, num_generations=3, temperature=1.0, top_p=0.9, max_new_tokens_per_seq=caps,
                               seed=seed)
        i, mk = o["completion_ids"].cpu(), o["masks"].cpu()
        return [i[q, :int(mk[q].sum())].tolist() for q in range(i.shape[0])]

    graphs_before = dict(eng._ctx.graphs)
    a = sampled(gen, 5)
    assert eng._ctx.graphs == graphs_before   # the same graph objects were replayed
    b = sampled(gen, 6)
    fresh = GRPOBatchGenerator(m, TinyTok(), chunk_size=16, max_decode_batch_size=96, verbose=False)
    assert sampled(fresh, 6) == b
    assert sampled(gen, 5) == a and a != b


def test_inline_prefill_in_slots_greedy(tiny):
    """Prompts prefilled in their own slots (``RolloutEngine.run_inline``, the path
    of BatchGenerator): 60 sequences through 5 slots, prompts of 1..40 tokens in
    chunks of 7 under a 23-token forward budget, per-sequence caps 1..9 (a cap of
    1 finishes a sequence at its first token, which frees its slot at once) and
    an EOS: every sequence equals the per-sequence reference loop
    (``scheduler_core.py:250-299, 445-600``).  A second run on the same engine
    (cached context, replayed graphs) gives the same tokens."""
    print("[case] inline prefill: 60 sequences / 5 slots greedy", flush=True)
    m, sd = tiny
    ps = prompts(60, 60, 1, 40)
    g = torch.Generator().manual_seed(61)
    caps = torch.randint(1, 10, (60,), generator=g).tolist()
    free = orl.scheduler_rollout(sd, ps, 9, max_valid_id=V - 4)
    eos = free[3][2]
    full = orl.scheduler_rollout(sd, ps, 9, eos=eos, max_valid_id=V - 4)
    ref = [r[:c] for r, c in zip(full, caps)]
    assert any(c == 1 for c in caps)
    assert any(r[-1] == eos and len(r) < c for r, c in zip(ref, caps)), "EOS path not exercised"
    eng = RolloutEngine(m, 5, eos_token_id=eos, max_valid_id=V - 4)
    for _ in range(2):
        res = eng.run_inline(ps, caps, temperature=0.0, chunk_size=7, max_batch_tokens=23, seed=3)
        assert res.tokens == ref
        assert res.timings["prefill_passes"] >= sum(len(p) for p in ps) // 23


def test_inline_sampled_streams_independent_of_slots_and_budget(tiny):
    """Sampled tokens of the inline path depend only on each sequence's prompt
    and (sequence, position) stream: 3, 17 and 40 slots with different chunk
    sizes and forward budgets (so different admission and prefill timing, row
    buckets and graph replays) give identical tokens; every sequence reaches its
    cap (no EOS)."""
    print("[case] inline prefill: sampled invariance", flush=True)
    m, _ = tiny
    ps = prompts(62, 40, 1, 30)
    runs = []
    for slots, chunk, budget in ((3, 5, 11), (17, 64, 4096), (40, 3, 7)):
        eng = RolloutEngine(m, slots, max_valid_id=V - 4)
        res = eng.run_inline(ps, 12, temperature=0.9, top_p=0.9, chunk_size=chunk, max_batch_tokens=budget, seed=7)
        runs.append(res.tokens)
    assert runs[0] == runs[1] == runs[2]
    assert all(len(t) == 12 for t in runs[0])


def test_batch_generator_bounded_memory_long_queue(tiny):
    """BatchGenerator over 2000 distinct prompts with 64 slots: the prompts are
    prefilled in the slots, so peak device memory does not grow with the queue
    (a prefilled state per prompt would add ~264 MB); greedy ids equal the
    reference loop on every 40th sequence."""
    print("[case] BatchGenerator 2000 prompts / 64 slots", flush=True)
    m, sd = tiny

    class Cfg:
        generation_max_batch_size = 64

    bg = BatchGenerator(m, TinyTok(), config=Cfg())

    def peak_for(n, seed):
        ps = prompts(seed, n, 2, 6)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        res = bg.generate(input_ids=ps, generation_config=GenerationConfig(max_length=3, temperature=0.0,
                                                                          chunk_size=4, max_batch_tokens=64))
        torch.cuda.synchronize()
        return ps, res, torch.cuda.max_memory_allocated() - base

    _, _, peak_small = peak_for(200, 40)
    ps, res, peak_big = peak_for(2000, 41)
    print(f"  peak extra memory: 200 prompts {peak_small / 2**20:.1f} MiB, 2000 prompts {peak_big / 2**20:.1f} MiB",
          flush=True)
    assert peak_big <= peak_small + (8 << 20)
    assert bool((res["masks"].sum(1) == 3).all())
    sub = list(range(0, 2000, 40))
    ref = orl.scheduler_rollout(sd, [ps[i] for i in sub], 3, max_valid_id=V - 4)
    for i, r in zip(sub, ref):
        assert res["completion_ids"][i].cpu().tolist() == r, i


def test_scheduler_graph_steps_equal_eager(tiny):
    """SchedulerCore's decode step replays a captured graph per row bucket (40
    slots: buckets of 32 and 40 rows as the pool fills and drains); its sampled
    tokens equal the eager launches' token for token, with per-sequence
    temperature / top_p / top_k, and both end every sequence at its cap."""
    print("[case] SchedulerCore graph vs eager decode", flush=True)
    m, _ = tiny
    ps = prompts(70, 90, 1, 20)
    runs = []
    for use_graph in (True, False):
        TokenSampler.manual_seed(77)
        sch = SchedulerCore(m, TinyTok(), max_batch_size=40, max_batch_tokens=64, prefill_chunk_size=8)
        sch.use_graph = use_graph
        seqs = [SequenceState(seq_id=i, prompt_tokens=p, max_new_tokens=5 + i % 7, temperature=0.8 + 0.01 * (i % 5),
                              top_p=0.9 if i % 2 else 1.0, top_k=30 if i % 3 == 0 else 0) for i, p in enumerate(ps)]
        sch.add_sequences(seqs)
        for _ in sch.run_to_completion_sync():
            pass
        if use_graph:
            assert set(sch._graphs.graphs) >= {32, 40}, sorted(sch._graphs.graphs)
        runs.append([s.generated_tokens for s in seqs])
        assert all(len(s.generated_tokens) == s.max_new_tokens for s in seqs)
    assert runs[0] == runs[1]
