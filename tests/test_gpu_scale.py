"""The bf16 decode and prefill paths at the benchmark models' real shapes, and
full-size rollouts with property checks.

* Layer shapes: two layers of the 1.5B preset (C=2048, H=32, LoRA 96/96/64/256)
  decoding 256 rows, and two layers of the 7.2B preset (C=4096, H=64, LoRA
  128/128/96/480) decoding 128 rows - the grouped packed-weight GEMM (split-K
  planes summed by the row kernels), the fused time-mix, and (C=4096) the
  1024-thread row kernels - against the float64 oracle (oracle/model.py) on the
  same bf16 weights.  Tolerance as for every bf16 model test: logits and each
  state tensor within 3e-2 relative (norm over the tensor).
* cfg4 in full (RWKV-7 1.5B, 64 prompts U(256, 2048) x 8 paths, temperature 1,
  top_p 0.95, Geometric(300) stop lengths): every path has exactly its stop
  length (max(cap, 2): the first token never ends a GRPO path), every id is a
  valid vocabulary id, two runs with 256 slots give bit-identical sampled
  streams (the race detector of the slot table at full size), and a run with
  128 slots has the same first tokens (drawn from the prefill logits) and the
  same per-path properties.  Streams at different slot counts are not compared
  bit for bit: the decode GEMM's K-split plan depends on the row count, so the
  float32 summation order - and, at temperature 1 on random weights, the drawn
  tokens - can differ in the last bits.
* Two 7.2B layers also decode 32, 64, 96 and 160 rows, and two 1.5B layers 48
  and 96: the other plans of the decode GEMM (32 x 32 tile with split K and the
  reduction launch; 64 x 64; 128 x 64 over a partial row tile; at C = 4096 and
  129-192 rows 64 x 64 over three row tiles; at C = 2048, 33-64 rows, 32 x 32
  without split and, 65-128 rows, 64 x 64 for the launches with epilogues).
* cfg5's model (RWKV-7 7.2B, all 32 layers) on a reduced rollout (8 prompts x
  2048 tokens, chunk 256): the same properties with 8 (twice) and 3 slots; and at
  its real slot count on the bench's own 128 x 2048-token prompts with the stop
  lengths cut to at most 128 tokens: two runs with 128 slots are bit-identical,
  every path has exactly its stop length and only valid ids.
"""

import pytest
import torch

from oracle import model as om
from rwkvtune_amd.grpo_batch_generator import GRPOBatchGenerator
from rwkvtune_amd.model import build_model, config_from_preset
from rwkvtune_amd.workloads import MAX_VALID_ID, cfg4_workload, cfg5_workload

pytestmark = pytest.mark.gpu

TOL = 3e-2


def rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def random_states(cfg, B, seed):
    g = torch.Generator().manual_seed(seed)
    C, H = cfg.n_embd, cfg.n_head
    return [{"att_x_prev": torch.randn(B, C, generator=g),
             "att_kv": torch.randn(B, H, 64, 64, generator=g) * 0.1,
             "ffn_x_prev": torch.randn(B, C, generator=g)} for _ in range(cfg.n_layer)]


def to_dev(states, dev):
    return [{k: v.to(dev) for k, v in s.items()} for s in states]


def to_f64(states):
    return [{k: v.double() for k, v in s.items()} for s in states]


@pytest.mark.parametrize("preset,rows,steps", [("rwkv7-1.5b", 256, 2), ("rwkv7-7.2b", 128, 1),
                                               ("rwkv7-7.2b", 32, 1), ("rwkv7-7.2b", 64, 1),
                                               ("rwkv7-7.2b", 96, 1), ("rwkv7-7.2b", 160, 1),
                                               ("rwkv7-1.5b", 48, 1), ("rwkv7-1.5b", 96, 1)])
def test_decode_layers_at_benchmark_shape(gpu_device, preset, rows, steps):
    print(f"[case] bf16 decode, two layers of {preset}, {rows} rows, {steps} steps", flush=True)
    cfg = config_from_preset(preset, n_layer=2, vocab_size=1000)
    m = build_model(cfg, dtype=torch.bfloat16, device="cuda", seed=77)
    assert m.use_grouped_gemm
    sd = om.cast_state_dict(m.state_dict(), torch.float64)
    st0 = random_states(cfg, rows, seed=78)
    st, ref_s = to_dev(st0, gpu_device), to_f64(st0)
    g = torch.Generator().manual_seed(79)
    for step in range(steps):
        tok = torch.randint(0, 1000, (rows, 1), generator=g)
        logits, st = m.forward_with_state(tok.to(gpu_device), st)
        ref_l, ref_s = om.forward_with_state(sd, tok, ref_s)
        e = rel(logits, ref_l)
        print(f"  step {step}: logits rel err {e:.3e}", flush=True)
        assert e <= TOL
        for l, (a, b) in enumerate(zip(st, ref_s)):
            for k in ("att_x_prev", "att_kv", "ffn_x_prev"):
                ek = rel(a[k], b[k])
                assert ek <= TOL, f"step {step} layer {l} {k}: rel err {ek:.3e}"


def test_prefill_layers_at_cfg4_shape(gpu_device):
    """Uniform [3, 70] prefill (library GEMMs, chunked matrix-core WKV, bf16
    operands) at the 1.5B shape, from random states, against the oracle."""
    print("[case] bf16 prefill, two layers of rwkv7-1.5b, 3 x 70 tokens", flush=True)
    cfg = config_from_preset("rwkv7-1.5b", n_layer=2, vocab_size=1000)
    m = build_model(cfg, dtype=torch.bfloat16, device="cuda", seed=80)
    sd = om.cast_state_dict(m.state_dict(), torch.float64)
    st0 = random_states(cfg, 3, seed=81)
    idx = torch.randint(0, 1000, (3, 70), generator=torch.Generator().manual_seed(82))
    logits, st = m.forward_with_state(idx.to(gpu_device), to_dev(st0, gpu_device))
    ref_l, ref_s = om.forward_with_state(sd, idx, to_f64(st0))
    assert rel(logits, ref_l) <= TOL
    for a, b in zip(st, ref_s):
        for k in ("att_x_prev", "att_kv", "ffn_x_prev"):
            assert rel(a[k], b[k]) <= TOL


class _Tok:
    def __init__(self):
        self.idx2token = {MAX_VALID_ID: b""}
        self.eos_token_id = None

    def decode(self, ids):
        return ""


def _rollout(gen, prompts, max_new, G, caps, seed):
    out = gen.generate(prompts, max_new, num_generations=G, temperature=1.0, top_p=0.95,
                       max_new_tokens_per_seq=caps, seed=seed)
    ids, masks = out["completion_ids"].cpu(), out["masks"].cpu()
    return [ids[q, :int(masks[q].sum())].tolist() for q in range(ids.shape[0])]


def _check_paths(paths, caps):
    for q, (p, c) in enumerate(zip(paths, caps)):
        assert len(p) == max(c, 2), (q, len(p), c)
        assert all(0 <= t <= MAX_VALID_ID for t in p), q


def test_cfg4_rollout_full_size_properties(gpu_device):
    print("[case] cfg4 full rollout: 1.5B, 512 paths, 256 vs 128 slots", flush=True)
    cfg = config_from_preset("rwkv7-1.5b")
    m = build_model(cfg, dtype=torch.bfloat16, device="cuda", seed=1234)
    prompts, caps = cfg4_workload()
    runs = []
    for slots in (256, 256, 128):
        gen = GRPOBatchGenerator(m, _Tok(), chunk_size=2048, max_decode_batch_size=slots, verbose=False)
        runs.append(_rollout(gen, prompts, 512, 8, caps, seed=99))
        print(f"  {slots} slots: {sum(len(p) for p in runs[-1])} tokens, "
              f"{gen.last_stats['decode_steps']} decode steps", flush=True)
        _check_paths(runs[-1], caps)
    assert runs[0] == runs[1]
    assert [p[0] for p in runs[0]] == [p[0] for p in runs[2]]


@pytest.fixture(scope="module")
def model_7b(gpu_device):
    cfg = config_from_preset("rwkv7-7.2b")
    return build_model(cfg, dtype=torch.bfloat16, device="cuda", seed=7272)


def test_cfg5_model_rollout_properties(model_7b):
    print("[case] cfg5 model (7.2B, 32 layers): 8 x 2048-token prompts, chunk 256, 8 vs 3 slots", flush=True)
    m = model_7b
    prompts, _ = cfg5_workload(n=8)
    caps = [c % 48 + 1 for c in cfg5_workload(n=8)[1]]
    runs = []
    for slots in (8, 8, 3):
        gen = GRPOBatchGenerator(m, _Tok(), chunk_size=256, max_decode_batch_size=slots, verbose=False)
        runs.append(_rollout(gen, prompts, 48, 1, caps, seed=5))
        _check_paths(runs[-1], caps)
    assert runs[0] == runs[1]
    assert [p[0] for p in runs[0]] == [p[0] for p in runs[2]]


def test_cfg5_rollout_128_slots_properties(model_7b):
    print("[case] cfg5 rollout at 128 slots: 128 x 2048-token prompts, chunk 256, caps <= 128, twice", flush=True)
    prompts, caps5 = cfg5_workload()
    caps = [min(c, 128) for c in caps5]
    assert len(prompts) == 128 and any(c < 128 for c in caps)
    gen = GRPOBatchGenerator(model_7b, _Tok(), chunk_size=256, max_decode_batch_size=128, verbose=False)
    runs = []
    for _ in range(2):
        runs.append(_rollout(gen, prompts, 128, 1, caps, seed=11))
        print(f"  {sum(len(p) for p in runs[-1])} tokens, {gen.last_stats['decode_steps']} decode steps", flush=True)
        _check_paths(runs[-1], caps)
    assert runs[0] == runs[1]
