#!/usr/bin/env python3
"""Benchmark of rwkvtune's batched-generation hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload rollout|cfg5|scheduler|decode|prefill|tmix|gemm|logprob|train|sampler]

Prints ONE JSON line.  One GPU only: ``--gpus N`` with N > 1 exits with a message.

Workloads
---------
rollout (default)  GRPO rollout on RWKV-7 1.5B (L=24, C=2048, H=32, V=65536), bf16
    weights from the seeded dense init, fp32 recurrent state: 64 random prompts of
    length U(256, 2048) x 8 generations = 512 sequences, temperature 1.0, top_p 0.95,
    at most 512 new tokens, per-sequence stop length ~ Geometric(mean 300) capped at
    512, 256 decode slots with continuous refill, through
    ``GRPOBatchGenerator.generate``.  A step is one whole rollout; value = generated
    tokens / wall time over the K timed rollouts (prefill, first token, decode and
    result assembly included).
cfg5               rollout on RWKV-7 7.2B (L=32, C=4096, H=64), bf16: 128 random 2048-token
    prompts, chunked prefill (chunk 256), up to 1024 sampled tokens (temperature 1.0,
    top_p 0.95) with Geometric(mean 600) stops, 128 slots; value = generated
    tokens / wall time of the rollout.  No CPU baseline (7.2B in fp32 on the host).
scheduler          cfg4's 512 sequences (the same prompts x 8 copies and stop caps)
    through ``BatchGenerator`` with 256 slots: no prompt sharing, each copy's prompt
    prefilled in its own slot when the device admits it into a freed slot
    (``RolloutEngine.run_inline``), ``TokenSampler.sample`` rules; value = generated
    tokens / wall time (prefill of every copy included).
logprob            GRPO log-prob recompute after a cfg4 rollout (RWKV-7 1.5B, bf16):
    512 sequences of 1024 prompt + 512 completion tokens through
    ``compute_per_token_logps``; a step is one whole batch; value = forward
    tokens/s; roofline = GEMM flops (block matrices at every position, head at
    the completion positions) per second against the 2.5 PFLOP/s bf16 peak.
train              WKV7 training operator (forward with 16-token checkpoints + backward,
    bf16) at one layer of a 1.5B training step: B=8 x T=4096 tokens, H=32; value =
    tokens/s of forward + backward; roofline = algorithmic HBM bytes of the
    backward kernel per second against 8 TB/s.
decode             isolated WKV7 decode kernel at B=256 slots, H=32 (cfg2); a step is
    one launch; value = algorithmic GB/s.
tmix               the fused decode time-mix kernel alone at the rollout shape, plus a
    plain copy of known size; for kernel-trace and PMC runs.
gemm               the decode projections alone (the roofline kernel of the default
    line) at --rows rows over the 1.5B model's 24 layers, plus a plain copy of
    known size; for kernel-trace and PMC runs.
prefill            chunked WKV7 prefill of cfg3 (64 ragged prompts ~U(64, 2048), H=32)
    in one launch; value = prompt tokens/s; roofline = bf16 MFMA rate executed
    (three part products per contraction) against the 2.5 PFLOP/s dense peak.

The default line also carries:
* ``roofline`` - the rollout's dominant kernel, the decode GEMM
  (``gemm_decode_kernel``, about half of the decode kernel time): the five grouped
  packed-weight launches of a layer at 256 rows over all 24 layers in turn (each
  layer's weights cold when reached), timed with HIP events on their launch stream;
  algorithmic bytes = the packed weights (activations are small and L2-resident);
  ``traffic`` = HBM bytes per launch from the committed PMC summary
  ``profiles/gemm_decode_m256_pmc.md``;
* ``roofline_tmix`` - the fused single-token time-mix (``tmix_decode_kernel``: WKV
  step + decay/LoRA element-wise + GroupNorm / bonus / gate, the second largest) at
  the rollout's shape (256 slots, H=32), rotating over 24 layer pools (3.2 GB) so no
  state is served from the 256 MB last-level cache; ``traffic`` from
  ``profiles/tmix_decode_cfg4_shape_pmc.md``;
* ``roofline_rollout`` - the whole rollout decode step: algorithmic bytes (every
  decode weight once per step + each live row's state read and written) over the
  measured decode time;
* ``wkv7_decode_cfg2`` / ``wkv7_prefill_cfg3`` - the stand-alone WKV kernels; for the
  prefill both the chunk algebra's contraction flops (``algorithmic_TFLOPs``,
  ``algorithmic_frac``) and the bf16 part products the MFMAs execute
  (``mfma_bf16_TFLOPs``, ``mfma_frac``: hi / lo operand splits, ~2.7x);
* ``cfg5_rollout`` - one timed 7.2B rollout (the ``cfg5`` workload) after one warm-up
  (``--no-cfg5`` skips it).

The CPU baseline is the reference's CPU path restated in ``oracle/`` (float32,
``torch.set_num_threads(os.cpu_count())``) timed on a bounded sample of the same
workload (rollout: one prompt's prefill forked to 256 paths plus decode steps).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import torch  # noqa: E402

from rwkvtune_amd.workloads import MAX_VALID_ID, cfg4_workload, cfg5_workload  # noqa: E402

PEAK_HBM_GBS = 8000.0          # MI355X datasheet HBM3E bandwidth
METRIC = "rollout tokens/s (RWKV7-1.5B, 512 seqs); WKV7 decode HBM GB/s vs peak"
N = 64
# algorithmic bytes per (slot, head) unit of one decode step
WKV_BYTES_PER_UNIT = 2 * N * N * 4 + 6 * N * 2 + N * 2          # state r+w, 6 bf16 inputs, bf16 y
TMIX_BYTES_PER_UNIT = 2 * N * N * 4 + 7 * N * 2 + N * 4 + N * 2  # state r+w, 7 bf16 inputs, fp32 v_first, bf16 out


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class NullTokenizer:
    """Synthetic-id tokenizer: decodable ids 0..65529 (the reference vocabulary's
    range), so 65530..65535 are banned as with the real tokenizer."""

    def __init__(self, max_id=MAX_VALID_ID):
        self.idx2token = {max_id: b""}
        self.eos_token_id = None

    def decode(self, ids):
        return ""


def time_launches(fn, n_iter, stream):
    """Average duration of fn() launches with HIP events on `stream`."""
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(n_iter):
        fn(i)
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / n_iter  # us


def pmc_traffic(path=os.path.join(ROOT, "profiles", "tmix_decode_cfg4_shape_pmc.md")):
    """HBM bytes per tmix_decode launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE in KiB per dispatch, each scaled by the same
    counter's reading for a plain copy of known size in the same run), or None."""
    import re
    try:
        text = open(path).read()
    except OSError:
        return None
    rows = {}
    for line in text.splitlines():
        m = re.match(r"\|\s*(.+?)\s*\|\s*([0-9.]+)\s*\|\s*([0-9.]+)\s*\|\s*$", line)
        if m:
            rows[m.group(1)] = (float(m.group(2)), float(m.group(3)))
    copy = next((v for k, v in rows.items() if k.startswith("plain copy")), None)
    kern = next((v for k, v in rows.items() if "tmix_decode_kernel" in k), None)
    m = re.search(r"plain copy of ([0-9,]+) B", text)
    if copy is None or kern is None or m is None:
        return None
    true_kib = int(m.group(1).replace(",", "")) / 1024.0
    return (kern[0] * true_kib / copy[0] + kern[1] * true_kib / copy[1]) * 1024


def gemm_pmc_traffic(path=os.path.join(ROOT, "profiles", "gemm_decode_m256_pmc.md")):
    """HBM bytes per decode-GEMM launch at 256 rows from the committed rocprofv3
    --pmc summary: its line 'Per layer (five launches): fabric reads R MB, writes
    W MB' (FETCH_SIZE and WRITE_SIZE, each scaled by the counter's reading for a
    plain copy of known size), divided by the five launches; or None."""
    import re
    try:
        text = open(path).read()
    except OSError:
        return None
    m = re.search(r"Per layer \(five launches\): fabric reads ([0-9.]+) MB, writes ([0-9.]+) MB", text)
    if m is None:
        return None
    return (float(m.group(1)) + float(m.group(2))) * 1e6 / 5


def head_pmc_traffic(path=os.path.join(ROOT, "profiles", "head_logits_m128_pmc.md")):
    """HBM bytes per head_logits_kernel launch at 128 rows (C = 2048) from the
    committed rocprofv3 --pmc summary: its line 'Per launch: fabric reads R MB,
    writes W MB' (FETCH_SIZE and WRITE_SIZE, each scaled by the counter's reading
    for a plain copy of known size); or None."""
    import re
    try:
        text = open(path).read()
    except OSError:
        return None
    m = re.search(r"Per launch: fabric reads ([0-9.]+) MB, writes ([0-9.]+) MB", text)
    if m is None:
        return None
    return (float(m.group(1)) + float(m.group(2))) * 1e6


def copy_reference(dev, n_bytes=256 * 32 * 64 * 64 * 4, reps=8):
    """Plain device copy of a known size (the PMC counters' scale reference)."""
    n = n_bytes // 4
    src = torch.ones(n, device=dev)
    dst = torch.zeros(n, device=dev)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    return n_bytes


def tmix_decode_leg(dev, iters=480, S=256, H=32, L=24):
    """Fused single-token time-mix at a rollout shape (default cfg4: 256 slots,
    H=32), L rotating layer pools."""
    from rwkvtune_amd import _lib
    from rwkvtune_amd.workloads import wkv_state
    C = H * N
    g = torch.Generator(device=dev).manual_seed(5)
    rnd = lambda *s: torch.randn(*s, generator=g, device=dev)
    r, k, v, wl, al, vl, gg = (rnd(S, C).to(torch.bfloat16) for _ in range(7))
    vfirst = rnd(S, C)
    params = [rnd(C) * 0.5 for _ in range(8)]
    ptrs = (__import__("ctypes").c_void_p * 8)(*[p.data_ptr() for p in params])
    pools = torch.randn((L, S, H, N, N), generator=g, device=dev) * 0.1
    row_slot = torch.arange(S, dtype=torch.int32, device=dev)
    out = torch.empty(S, C, dtype=torch.bfloat16, device=dev)
    P = _lib.ptr
    st = torch.cuda.current_stream(dev)

    def launch(i):
        _lib.call("rwkv7_tmix_decode", 2, S, H, 0, P(r), P(k), P(v), P(wl), P(al), P(vl), P(gg), P(vfirst),
                  ptrs, P(pools[i % L]), S, P(row_slot), P(out), _lib.stream_of(out))
    for i in range(48):
        launch(i)
    us = time_launches(launch, iters, st)
    units = S * H
    gbs = units * TMIX_BYTES_PER_UNIT / (us * 1e-6) / 1e9
    return {"kernel": "tmix_decode_kernel<bf16> (fused WKV decode time-mix)", "slots": S, "H": H, "pools": L,
            "us_per_launch": us, "bytes_per_launch": units * TMIX_BYTES_PER_UNIT, "GBs": gbs,
            "frac": gbs / PEAK_HBM_GBS, "launches": iters}


def gemm_decode_leg(model, dev, M=256, reps=10):
    """The decode step's projections on the packed-weight grouped GEMM, exactly
    as forward_pooled issues them (r/k/v + LoRA downs, LoRA ups, output
    projection partials, FFN key with relu^2, FFN value partials), at M rows,
    over all layers in turn (each layer's weights are cold when reached).
    Algorithmic bytes = the packed weights' N x K x 2 per layer (activations are
    small and L2-resident); HIP events on the launch stream."""
    from rwkvtune_amd import _lib
    from rwkvtune_amd.model import RWKV7Model
    packs = model.packs()
    C = model.config.n_embd
    dt = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(9)
    mixes = torch.randn((7, M, C), generator=g, device=dev).to(dt)
    rkv = torch.empty((3, M, C), dtype=dt, device=dev)
    o = torch.randn((M, C), generator=g, device=dev).to(dt)
    xk = torch.randn((M, C), generator=g, device=dev).to(dt)
    st = torch.cuda.current_stream(dev)
    stream = _lib.stream_of(o)
    bufs = {}

    def layer(l):
        pk = packs[l]
        gp = pk.gp
        nl, D = pk.lora_down.shape[0], pk.lora_down.shape[2]
        if (nl, D) not in bufs:
            bufs[(nl, D)] = (torch.zeros((nl, M, D), dtype=dt, device=dev), torch.empty((nl, M, C), dtype=dt, device=dev))
        h, up = bufs[(nl, D)]
        xr, xkk, xv, xw, xa, xg, _ = mixes.unbind(0)
        dn = [("w1", 0, 2), ("a1", 1, 0), ("g1", 2, 3)] + ([] if l == 0 else [("v1", 3, 0)])
        src = {"w1": xw, "a1": xa, "g1": xg, "v1": xv}
        probs = [(xr, gp["r"], rkv[0], 0), (xkk, gp["k"], rkv[1], 0), (xv, gp["v"], rkv[2], 0)]
        probs += [(src[n], gp[n], h[i, :, :gp[n].N], e) for n, i, e in dn]
        RWKV7Model._gemm_group(M, probs, stream)
        ups = [("w2", 0), ("a2", 1), ("g2", 2)] + ([] if l == 0 else [("v2", 3)])
        RWKV7Model._gemm_group(M, [(h[i, :, :gp[n].K], gp[n], up[i], 0) for n, i in ups], stream)
        RWKV7Model._gemm_partials(M, o, gp["o"], stream)
        hk = bufs.setdefault("hk", torch.empty((M, gp["fk"].N), dtype=dt, device=dev))
        RWKV7Model._gemm_group(M, [(xk, gp["fk"], hk, 1)], stream)
        RWKV7Model._gemm_partials(M, hk, gp["fv"], stream)

    L = len(packs)
    for l in range(L):
        layer(l)
    us = time_launches(lambda i: layer(i % L), reps * L, st)
    wbytes = sum(sum(w.N * w.K * 2 for w in pk.gp.values()) for pk in packs) / L
    gbs = wbytes / (us * 1e-6) / 1e9
    return {"kernel": "gemm_decode_kernel (5 grouped launches per layer)", "M": M, "us_per_layer": us,
            "weight_bytes_per_layer": wbytes, "GBs": gbs, "frac": gbs / PEAK_HBM_GBS}


def wkv_decode_leg(dev, iters=800, pools_n=8):
    """Stand-alone WKV7 decode kernel, cfg2 shape, rotating over `pools_n` pools."""
    from rwkvtune_amd import operators as ops
    from rwkvtune_amd.workloads import wkv_inputs, wkv_state
    B, H = 256, 32
    inp = wkv_inputs((B,), H, N, seed=1000).to(dev)
    pools = [wkv_state(B, H, N, seed=1001 + i).to(dev) for i in range(pools_n)]
    y = torch.empty_like(inp.r)
    args = inp.as_tuple()
    st = torch.cuda.current_stream(dev)
    for i in range(50):
        ops.wkv7_decode(pools[i % pools_n], None, *args, y=y)
    us = time_launches(lambda i: ops.wkv7_decode(pools[i % pools_n], None, *args, y=y), iters, st)
    units = B * H
    gbs = units * WKV_BYTES_PER_UNIT / (us * 1e-6) / 1e9
    return {"kernel": "wkv7_seq_kernel<bf16> (T=1)", "B": B, "H": H, "us_per_step": us,
            "bytes_per_step": units * WKV_BYTES_PER_UNIT, "GBs": gbs, "frac": gbs / PEAK_HBM_GBS,
            "pools": pools_n, "launches": iters}


# chunked prefill (L = 32 tokens, N = 64): contraction flops per (chunk, head) of the
# matrix form - A_ab, A_ak, B_rb, B_rk (4 x L*L*N), S a~^T and S r~^T (2 x N*L*N),
# V^T A_ak (N*L*L), SA B_rb + V^T B_rk (2 x N*L*L), SA bbar + V^T kbar (2 x N*L*N).
# Executed as bf16 MFMA part products on hi/lo operand splits: 3 per contraction, 2 for
# the three products with V when the inputs are bf16 (V is exact in bf16: no lo part)
CHUNK_L = 32
PREFILL_V_FLOPS_PER_CHUNK_HEAD = 2 * (2 * N * CHUNK_L * CHUNK_L + N * CHUNK_L * N)
PREFILL_FLOPS_PER_CHUNK_HEAD = 2 * (4 * CHUNK_L * CHUNK_L * N + 2 * N * CHUNK_L * N + N * CHUNK_L * CHUNK_L
                                    + 2 * N * CHUNK_L * CHUNK_L + 2 * N * CHUNK_L * N)
PREFILL_MFMA_FLOPS_PER_CHUNK_HEAD = 3 * PREFILL_FLOPS_PER_CHUNK_HEAD - PREFILL_V_FLOPS_PER_CHUNK_HEAD
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
PREFILL_BYTES_PER_HEAD_TOKEN = 7 * N * 2        # r, w, k, v, a, b in, y out (bf16)
STATE_BYTES_PER_SEQ_HEAD = 2 * N * N * 4        # fp32 state read + write


def cfg3_lengths():
    from rwkvtune_amd.workloads import ragged_lengths
    return ragged_lengths(64, 64, 2048, seed=3)


def prefill_leg(dev, iters=20, chunk_len=64):
    """cfg3: ragged chunked prefill, 64 prompts ~U(64, 2048), H=32, bf16 inputs drawn
    as in cfg2, zero initial state; one launch covers the whole batch."""
    from rwkvtune_amd import operators as ops
    from rwkvtune_amd.workloads import cu_seqlens_of, wkv_inputs
    H = 32
    lens = cfg3_lengths()
    cu = cu_seqlens_of(lens)
    total = cu[-1]
    inp = wkv_inputs((total,), H, N, seed=115).to(dev)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=dev)
    pool = torch.zeros(len(lens), H, N, N, device=dev)
    y = torch.empty_like(inp.r)
    args = inp.as_tuple()
    st = torch.cuda.current_stream(dev)

    def launch(i, cl=chunk_len):
        pool.zero_()
        ops.wkv7_prefill(pool, None, cu_d, *args, y=y, chunk_len=cl)
    # the zero fill is timed separately and taken out
    for i in range(3):
        launch(i)
    us_total = time_launches(launch, iters, st)
    us_fill = time_launches(lambda i: pool.zero_(), iters, st)
    us = us_total - us_fill
    us_serial = time_launches(lambda i: launch(i, 1), 3, st) - us_fill
    chunks = sum((n + CHUNK_L - 1) // CHUNK_L for n in lens) * H
    flops = chunks * PREFILL_FLOPS_PER_CHUNK_HEAD
    nbytes = total * H * PREFILL_BYTES_PER_HEAD_TOKEN + len(lens) * H * STATE_BYTES_PER_SEQ_HEAD
    alg_tf = flops / (us * 1e-6) / 1e12
    mfma_tf = chunks * PREFILL_MFMA_FLOPS_PER_CHUNK_HEAD / (us * 1e-6) / 1e12
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"kernel": "wkv7_chunk_kernel<bf16>", "tokens": total, "seqs": len(lens), "H": H,
            "us_per_launch": us, "tokens_per_s": total / (us * 1e-6), "algorithmic_TFLOPs": alg_tf,
            "mfma_bf16_TFLOPs": mfma_tf, "mfma_frac": mfma_tf / PEAK_BF16_TFLOPS,
            "flops_per_launch": flops, "bytes_per_launch": nbytes, "GBs": gbs, "hbm_frac": gbs / PEAK_HBM_GBS,
            "token_serial_us": us_serial, "speedup_vs_token_serial": us_serial / us, "launches": iters}


def cpu_baseline_prefill(max_tokens=2048):
    """The reference CPU operator (restated in oracle/) over the first cfg3 prompts."""
    from oracle.wkv7 import wkv7_cpu
    from rwkvtune_amd.workloads import wkv_inputs
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    H = 32
    lens = cfg3_lengths()
    n = lens[0]
    n = min(n, max_tokens)
    inp = wkv_inputs((1, n), H, N, seed=115)
    S0 = torch.zeros(1, H, N, N)
    t0 = time.perf_counter()
    wkv7_cpu(*(t.float() for t in inp.as_tuple()), N, S0)
    dt = time.perf_counter() - t0
    return {"value": n / dt, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"first cfg3 prompt ({n} tokens, H=32) through the restated wkv_cpu.py path, fp32; "
                      f"{dt:.2f} s"}


def rollout(steps, warmup, dev):
    from rwkvtune_amd.grpo_batch_generator import GRPOBatchGenerator
    from rwkvtune_amd.model import build_model, config_from_preset
    cfg = config_from_preset("rwkv7-1.5b")
    log("[bench] building RWKV-7 1.5B (bf16, seeded dense init) ...")
    model = build_model(cfg, dtype=torch.bfloat16, device=dev, seed=1234)
    prompts, caps = cfg4_workload()
    tok = NullTokenizer()
    gen = GRPOBatchGenerator(model, tok, chunk_size=2048, max_decode_batch_size=256, eos_token_id=None,
                             verbose=False)
    kw = dict(max_new_tokens=512, num_generations=8, temperature=1.0, top_p=0.95, top_k=0,
              max_new_tokens_per_seq=caps)
    # warm-up: one small rollout (kernels, GEMM heuristics, graph capture), then W full ones
    gen.generate(prompts[:2], 8, num_generations=4, temperature=1.0, top_p=0.95)
    for i in range(warmup):
        log(f"[bench] warm-up rollout {i + 1}/{warmup}")
        gen.generate(prompts, **kw)
    torch.cuda.synchronize(dev)
    total_gen, total_s, stats = 0, 0.0, []
    for i in range(steps):
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        out = gen.generate(prompts, **kw)
        torch.cuda.synchronize(dev)
        dt = time.perf_counter() - t0
        n_gen = int(out["masks"].sum())
        total_gen += n_gen
        total_s += dt
        st = dict(gen.last_stats)
        stats.append(st)
        log(f"[bench] rollout {i + 1}/{steps}: {n_gen} tokens in {dt:.3f} s = {n_gen / dt:.0f} tok/s "
            f"(prefill {st['prefill_s']:.3f}s, decode {st['decode_s']:.3f}s, {st['decode_steps']} steps)")
    return model, prompts, caps, {"tokens": total_gen, "seconds": total_s, "value": total_gen / total_s,
                                  "ms_per_step": total_s / steps * 1e3, "runs": stats}


def scheduler_rollout(steps, warmup, dev, max_batch_tokens=16384, chunk_size=2048):
    """cfg4's 512 sequences (64 prompts x 8 copies, the same caps) through
    ``BatchGenerator`` with 256 slots: every copy's prompt is prefilled in its own
    slot as it is admitted (the reference's BatchGenerator / SchedulerCore
    semantics, no prompt sharing), ``TokenSampler.sample`` rules, temp 1.0,
    top_p 0.95."""
    from rwkvtune_amd.batch_generator import BatchGenerator, GenerationConfig
    from rwkvtune_amd.model import build_model, config_from_preset
    cfg = config_from_preset("rwkv7-1.5b")
    log("[bench] building RWKV-7 1.5B (bf16, seeded dense init) ...")
    model = build_model(cfg, dtype=torch.bfloat16, device=dev, seed=1234)
    prompts, caps = cfg4_workload()

    class Cfg:
        generation_max_batch_size = 256

    bg = BatchGenerator(model, NullTokenizer(), config=Cfg())
    gc = GenerationConfig(max_length=512, temperature=1.0, top_p=0.95, num_generations=8,
                          max_batch_tokens=max_batch_tokens, chunk_size=chunk_size)
    bg.generate(input_ids=prompts[:2], generation_config=GenerationConfig(max_length=8, temperature=1.0, top_p=0.95,
                                                                          num_generations=4))
    for i in range(warmup):
        log(f"[bench] scheduler warm-up {i + 1}/{warmup}")
        bg.generate(input_ids=prompts, generation_config=gc, max_new_tokens_per_seq=caps)
    total_gen, total_s, stats = 0, 0.0, []
    for i in range(steps):
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        out = bg.generate(input_ids=prompts, generation_config=gc, max_new_tokens_per_seq=caps)
        torch.cuda.synchronize(dev)
        dt = time.perf_counter() - t0
        n_gen = int(out["masks"].sum())
        total_gen += n_gen
        total_s += dt
        st = dict(bg.last_stats)
        stats.append(st)
        log(f"[bench] scheduler rollout {i + 1}/{steps}: {n_gen} tokens in {dt:.3f} s = {n_gen / dt:.0f} tok/s "
            f"({st['prompt_tokens']} prompt tokens prefilled in {st['prefill_passes']} passes, "
            f"{st['decode_steps']} decode steps)")
    return {"tokens": total_gen, "seconds": total_s, "value": total_gen / total_s,
            "ms_per_step": total_s / steps * 1e3, "runs": stats, "prompt_tokens": stats[-1]["prompt_tokens"]}


def rollout_roofline(model, ro, n_paths):
    """Algorithmic HBM bytes of the rollout's decode steps over their measured
    time: every step reads each decode weight once (the packed projections and
    the LM head), and every live row reads and writes its recurrent state (WKV
    state 2 x L x H x 64 x 64 x 4 B, x_prev rows 4 x L x C x 4 B).  Live rows
    summed over the steps = tokens made by decode steps = generated tokens minus
    the first token of each path (drawn from the prefill logits)."""
    cfg = model.config
    packs = model.packs()
    w_step = sum(sum(w.N * w.K * 2 for w in pk.gp.values()) for pk in packs)
    w_step += cfg.vocab_size * cfg.n_embd * 2
    row = 2 * cfg.n_layer * cfg.n_head * 64 * 64 * 4 + 4 * cfg.n_layer * cfg.n_embd * 4
    run = ro["runs"][-1]
    steps, dec_s = run["decode_steps"], run["decode_s"]
    live_rows = run["generated_tokens"] - n_paths
    total = steps * w_step + live_rows * row
    gbs = total / dec_s / 1e9
    return {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
            "ms_per_step": dec_s / steps * 1e3, "weight_bytes_per_step": w_step, "state_bytes_per_live_row": row,
            "decode_steps": steps, "live_rows": live_rows, "bytes": total}


def rollout_cfg5(steps, warmup, dev):
    """cfg5: RWKV-7 7.2B (bf16, seeded dense init), 128 prompts x 2048 tokens,
    chunked prefill (chunk 256), up to 1024 sampled tokens per sequence (temp 1.0,
    top_p 0.95) with Geometric(600) stops, all 128 sequences in slots at once."""
    from rwkvtune_amd.grpo_batch_generator import GRPOBatchGenerator
    from rwkvtune_amd.model import build_model, config_from_preset
    cfg = config_from_preset("rwkv7-7.2b")
    log("[bench] building RWKV-7 7.2B (bf16, seeded dense init) ...")
    model = build_model(cfg, dtype=torch.bfloat16, device=dev, seed=7272)
    prompts, caps = cfg5_workload()
    gen = GRPOBatchGenerator(model, NullTokenizer(), chunk_size=256, max_decode_batch_size=128,
                             eos_token_id=None, verbose=False)
    kw = dict(max_new_tokens=1024, num_generations=1, temperature=1.0, top_p=0.95, top_k=0,
              max_new_tokens_per_seq=caps)
    gen.generate(prompts[:2], 8, num_generations=1, temperature=1.0, top_p=0.95)
    for i in range(warmup):
        log(f"[bench] cfg5 warm-up rollout {i + 1}/{warmup}")
        gen.generate(prompts, **kw)
    total_gen, total_s, stats = 0, 0.0, []
    for i in range(steps):
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        out = gen.generate(prompts, **kw)
        torch.cuda.synchronize(dev)
        dt = time.perf_counter() - t0
        n_gen = int(out["masks"].sum())
        total_gen += n_gen
        total_s += dt
        st = dict(gen.last_stats)
        stats.append(st)
        log(f"[bench] cfg5 rollout {i + 1}/{steps}: {n_gen} tokens in {dt:.3f} s = {n_gen / dt:.0f} tok/s "
            f"(prefill {st['prefill_s']:.3f}s, decode {st['decode_s']:.3f}s, {st['decode_steps']} steps)")
    return {"tokens": total_gen, "seconds": total_s, "value": total_gen / total_s,
            "ms_per_step": total_s / steps * 1e3, "runs": stats, "prompt_tokens": sum(len(p) for p in prompts)}


def logprob_workload(seed=6, B=512, P=1024, C=512, V=65536):
    g = torch.Generator().manual_seed(seed)
    prompt = torch.randint(1, MAX_VALID_ID + 1, (B // 8, P), generator=g).repeat_interleave(8, 0)
    completion = torch.randint(1, MAX_VALID_ID + 1, (B, C), generator=g)
    return prompt, completion


def matrix_macs(model):
    """Multiply-adds per token of the blocks' matrices (projections, LoRAs, FFN)."""
    return sum(p.numel() for n, p in model.named_parameters()
               if p.ndim == 2 and n not in ("emb.weight", "head.weight") and not n.endswith(".r_k"))


def logprob_recompute(steps, warmup, dev):
    """GRPO log-prob recompute after a cfg4-sized rollout: 512 sequences (64 prompts
    x 8 generations) of 1024 prompt + 512 completion tokens on RWKV-7 1.5B, through
    ``compute_per_token_logps`` (forward over prompt + completion[:-1] padded to
    1536, ln_out + head + selective log-softmax at the 512 completion positions)."""
    from rwkvtune_amd.grpo_utils import compute_per_token_logps
    from rwkvtune_amd.model import build_model, config_from_preset
    cfg = config_from_preset("rwkv7-1.5b", ctx_len=2048)
    log("[bench] building RWKV-7 1.5B (bf16, seeded dense init) ...")
    model = build_model(cfg, dtype=torch.bfloat16, device=dev, seed=1234)
    prompt, completion = logprob_workload()
    prompt, completion = prompt.to(dev), completion.to(dev)
    B, P = prompt.shape
    C = completion.shape[1]
    T = -(-(P + C - 1) // 16) * 16
    compute_per_token_logps(model, prompt[:16, :64], completion[:16, :16])
    for i in range(warmup):
        compute_per_token_logps(model, prompt, completion)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for i in range(steps):
        out = compute_per_token_logps(model, prompt, completion)
    torch.cuda.synchronize(dev)
    dt = (time.perf_counter() - t0) / steps
    assert out.shape == (B, C) and bool(torch.isfinite(out).all())
    macs = matrix_macs(model)
    flops = 2.0 * macs * B * T + 2.0 * cfg.n_embd * cfg.vocab_size * B * C
    log(f"[bench] logprob recompute: {dt:.3f} s per batch, {B * T / dt:.0f} forward tok/s, "
        f"{flops / dt / 1e12:.0f} TFLOP/s of GEMM work")
    return model, {"seconds": dt, "tokens": B * T, "value": B * T / dt, "completion_tokens": B * C,
                   "gemm_TFLOPs": flops / dt / 1e12, "flops": flops, "T": T}


def cpu_baseline_logprob(model, P=1024, C=512):
    """The restated reference recompute (oracle/logprob.py, fp32) for one sequence."""
    from oracle import logprob as olp
    from oracle import model as om
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    sd = om.cast_state_dict(model.state_dict(), torch.float32)
    prompt, completion = logprob_workload()
    pr, co = prompt[:1, :P], completion[:1, :C]
    t0 = time.perf_counter()
    olp.per_token_logps(sd, pr, co, ctx_len=model.config.ctx_len, dtype=torch.float32)
    dt = time.perf_counter() - t0
    T = -(-(P + C - 1) // 16) * 16
    return {"value": T / dt, "unit": "forward tokens/s", "cores": cores, "kind": "port",
            "sample": f"one sequence of {P} prompt + {C} completion tokens ({T} forward tokens) through the "
                      f"restated reference recompute (fp32 forward, full logits, selective log-softmax); "
                      f"{dt:.1f} s"}


# algorithmic bytes per (token, head) of the training operator: forward reads 6 bf16
# inputs and writes y (bf16), sa (fp32) and the 16-token checkpoints (16 KB / 16);
# backward reads 7 bf16 inputs, sa and the checkpoints and writes 6 bf16 gradients
TRAIN_FWD_BYTES = 6 * N * 2 + N * 2 + N * 4 + N * N * 4 // 16
TRAIN_BWD_BYTES = 7 * N * 2 + N * 4 + N * N * 4 // 16 + 6 * N * 2


def train_leg(dev, steps, warmup, B=8, T=4096, H=32):
    """WKV7 training operator (forward + backward, bf16) at one layer of a 1.5B
    training step on B x T tokens; HIP events around each kernel."""
    from rwkvtune_amd import operators as ops
    g = torch.Generator(device=dev).manual_seed(21)
    shp = (B, T, H, N)
    r, k, v = (torch.randn(shp, generator=g, device=dev).bfloat16() for _ in range(3))
    w = (torch.rand(shp, generator=g, device=dev) * -5.5 - 0.5).bfloat16()
    kk = torch.nn.functional.normalize(torch.randn(shp, generator=g, device=dev), dim=-1)
    a, b = (-kk).bfloat16(), (kk * torch.rand(shp, generator=g, device=dev)).bfloat16()
    dy = torch.randn(shp, generator=g, device=dev).bfloat16()
    st = torch.cuda.current_stream(dev)
    for _ in range(warmup):
        _, ck, sa = ops._train_forward(w, r, k, v, a, b)
        ops._train_backward(w, r, k, v, a, b, dy, ck, sa)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    fwd = bwd = 0.0
    for _ in range(steps):
        ev[0].record(st)
        _, ck, sa = ops._train_forward(w, r, k, v, a, b)
        ev[1].record(st)
        ops._train_backward(w, r, k, v, a, b, dy, ck, sa)
        ev[2].record(st)
        ev[2].synchronize()
        fwd += ev[0].elapsed_time(ev[1]) / steps
        bwd += ev[1].elapsed_time(ev[2]) / steps
    units = B * T * H
    fgbs = units * TRAIN_FWD_BYTES / (fwd * 1e-3) / 1e9
    bgbs = units * TRAIN_BWD_BYTES / (bwd * 1e-3) / 1e9
    return {"fwd_ms": fwd, "bwd_ms": bwd, "tokens_per_s": B * T / ((fwd + bwd) * 1e-3), "fwd_GBs": fgbs,
            "bwd_GBs": bgbs, "B": B, "T": T, "H": H,
            "kernels": "wkv7_chunk2_kernel<bf16, train> (chunked forward), wkv7_train_bwd_kernel<bf16>"}


def cpu_baseline_train(T=64, H=32):
    """The reference's CPU path for training (the restated wkv_cpu.py recurrence,
    float32, with torch autograd for the backward) on one sequence of T tokens."""
    from oracle.wkv7 import wkv7_cpu
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(3)
    C = H * N
    xs = [torch.randn(1, T, C, generator=g) for _ in range(6)]
    xs[1] = torch.rand(1, T, C, generator=g) * -5.5 - 0.5
    xs = [x.requires_grad_(True) for x in xs]
    t0 = time.perf_counter()
    y, _ = wkv7_cpu(*xs, N)
    y.sum().backward()
    dt = time.perf_counter() - t0
    return {"value": T / dt, "unit": "tokens/s (forward + backward, one layer)", "cores": cores, "kind": "port",
            "sample": f"one sequence of {T} tokens, H={H}, through the restated wkv_cpu.py recurrence (fp32) "
                      f"and torch autograd; {dt:.1f} s"}


def cpu_baseline_rollout(model, prompts, paths=256, decode_steps=2):
    """The reference CPU rollout (oracle/: fp32 forward_with_state, batched
    sample_batch rules) on a bounded sample: one prompt prefilled, forked to
    `paths` generation paths, first token, then `decode_steps` lockstep steps."""
    from oracle import model as om
    from oracle import sampler as osm
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    sd = om.cast_state_dict(model.state_dict(), torch.float32)
    p = prompts[0][:512]
    g = torch.Generator().manual_seed(0)
    t0 = time.perf_counter()
    lg, st = om.forward_with_state(sd, torch.tensor([p]), None, torch.float32)
    t1 = time.perf_counter()
    states = [{k: v.expand(paths, *v.shape[1:]).clone() for k, v in layer.items()} for layer in st]
    tok, _ = osm.sample_batch_torch(lg[:, -1].expand(paths, -1), 1.0, 0.95, 0, MAX_VALID_ID, g)
    generated = paths
    for _ in range(decode_steps):
        lg, states = om.forward_with_state(sd, tok[:, None], states, torch.float32)
        tok, _ = osm.sample_batch_torch(lg[:, -1], 1.0, 0.95, 0, MAX_VALID_ID, g)
        generated += paths
    t2 = time.perf_counter()
    wall = t2 - t0
    return {"value": generated / wall, "unit": "tokens/s", "cores": cores, "kind": "port",
            "prefill_tok_s": len(p) / (t1 - t0), "decode_tok_s": paths * decode_steps / (t2 - t1),
            "sample": (f"GRPO rollout sample on the restated reference CPU path (fp32): prefill of one "
                       f"{len(p)}-token prompt ({t1 - t0:.1f} s), fork to {paths} paths, first token + "
                       f"{decode_steps} lockstep decode steps ({t2 - t1:.1f} s); {generated} generated tokens "
                       f"in {wall:.1f} s; prefill {len(p) / (t1 - t0):.0f} tok/s, decode "
                       f"{paths * decode_steps / (t2 - t1):.0f} tok/s")}


def cpu_baseline_decode(reps: int = 3):
    """The reference CPU operator (restated in oracle/) for one cfg2 step, fp32."""
    from oracle.wkv7 import wkv7_cpu
    from rwkvtune_amd.workloads import wkv_inputs, wkv_state
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    B, H = 256, 32
    inp = wkv_inputs((B, 1), H, N, seed=1000)
    S0 = wkv_state(B, H, N, seed=1001)
    wkv7_cpu(*inp.as_tuple(), N, S0)
    t0 = time.perf_counter()
    for _ in range(reps):
        wkv7_cpu(*inp.as_tuple(), N, S0)
    dt = (time.perf_counter() - t0) / reps
    gbs = B * H * WKV_BYTES_PER_UNIT / dt / 1e9
    return {"value": gbs, "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"one cfg2 decode step (B=256, H=32) through the restated wkv_cpu.py path, fp32, "
                      f"mean of {reps}; {dt * 1e3:.1f} ms/step"}


def head_sampler_leg(dev, M=256, reps=200, C=2048):
    """One sampling step of the cfg4 rollout at M rows: the LM head as the model
    computes it (the library's head GEMM over the packed head up to
    HeadPack.MAX_ROWS rows, hipBLASLt above; [M, C] x [65536, C]^T bf16, two head
    copies alternating so the 268 MB weight is not cache-resident, as in the
    rollout where the layers' weights stream in between) and the sampler (one
    16-bit sampling launch, RULE_BATCH, temperature 1, top_p 0.95, ids above 65529
    banned), as graph replays; HIP events on the launch stream.  The library
    GEMM's head time at the same M is reported beside it."""
    import torch.nn.functional as F
    from rwkvtune_amd import sampler as dsm
    from rwkvtune_amd.model import HeadPack
    V = 65536
    g = torch.Generator(device=dev).manual_seed(11)
    heads = [(torch.randn(V, C, generator=g, device=dev) * 0.02).to(torch.bfloat16) for _ in range(2)]
    packs = [HeadPack(w) for w in heads]
    xo = torch.randn(M, C, generator=g, device=dev).to(torch.bfloat16)
    logits = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
    buf = dsm.SamplerBuffers(M, dev)
    buf.set_uniform(1.0, 0.95, 0)
    buf.rng_key.copy_(torch.arange(M, device=dev))
    tok = torch.empty(M, dtype=torch.int64, device=dev)
    lp = torch.empty(M, dtype=torch.float32, device=dev)

    def head_lib(i):
        torch.matmul(xo, heads[i % 2].t(), out=logits)

    def head(i):
        if M <= HeadPack.MAX_ROWS:
            packs[i % 2].logits(xo, out=logits)
        else:
            head_lib(i)

    def sample(i):  # a fixed counter: the same draws every step, the same work
        dsm.sample_rows(logits, buf, rule=dsm.RULE_BATCH, max_valid_id=MAX_VALID_ID, seed=1, out_tok=tok,
                        out_logp=lp)

    res = {}
    s = torch.cuda.Stream(dev)
    for name, fns in (("head", (head,)), ("head_lib", (head_lib,)), ("sampler", (sample,)),
                      ("step", (head, sample))):
        with torch.cuda.stream(s):
            for i in range(2):
                for f in fns:
                    f(i)
            torch.cuda.synchronize(dev)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=s):
                for i in range(20):
                    for f in fns:
                        f(i)
            graph.replay()  # the first replay uploads the graph
            torch.cuda.synchronize(dev)
            res[name] = time_launches(lambda i: graph.replay(), reps // 20, s) / 20
    wbytes = V * C * 2
    return {"M": M, "head_us": res["head"], "head_lib_us": res["head_lib"], "sampler_us": res["sampler"],
            "step_us": res["step"], "head_GBs": wbytes / (res["head"] * 1e-6) / 1e9, "logits_bytes": M * V * 2,
            "tokens_per_s": M / (res["step"] * 1e-6), "head_kernel": M <= HeadPack.MAX_ROWS,
            "valid": bool(((tok >= 0) & (tok <= MAX_VALID_ID)).all())}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="rollout",
                    choices=["rollout", "cfg5", "scheduler", "decode", "prefill", "tmix", "gemm", "logprob",
                             "train", "sampler"])
    ap.add_argument("--rows", type=int, default=256, help="rows of the gemm and sampler workloads")
    ap.add_argument("--embd", type=int, default=2048, help="head input width of the sampler workload (4096: 7.2B)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-cfg5", action="store_true", help="skip the 7.2B rollout leg of the default workload")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {a.gpus}): this build measures one GPU's "
              "share; the rollout shards by sequence with no cross-GPU exchange",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    from rwkvtune_amd import _lib
    _lib.load()

    if a.workload == "rollout":
        steps = 3 if a.steps is None else a.steps
        warmup = 1 if a.warmup is None else a.warmup
        model, prompts, caps, ro = rollout(steps, warmup, dev)
        log("[bench] fused decode time-mix kernel (roofline) ...")
        tm = tmix_decode_leg(dev)
        log(f"[bench] tmix_decode: {tm['us_per_launch']:.2f} us/launch, {tm['GBs']:.0f} GB/s")
        wk = wkv_decode_leg(dev)
        log(f"[bench] wkv7 decode cfg2: {wk['us_per_step']:.2f} us/step, {wk['GBs']:.0f} GB/s")
        pf = prefill_leg(dev)
        log(f"[bench] wkv7 chunked prefill cfg3: {pf['us_per_launch']:.0f} us, {pf['mfma_bf16_TFLOPs']:.0f} "
            f"bf16 MFMA TFLOP/s, {pf['speedup_vs_token_serial']:.2f}x token-serial")
        gm = gemm_decode_leg(model, dev)
        log(f"[bench] decode GEMM (M=256): {gm['us_per_layer']:.1f} us/layer, {gm['GBs']:.0f} GB/s of weights")
        rr = rollout_roofline(model, ro, n_paths=len(caps))
        log(f"[bench] rollout decode step: {rr['ms_per_step']:.3f} ms, {rr['achieved']:.0f} GB/s algorithmic")
        cpu = None
        if not a.no_cpu_baseline:
            log("[bench] cpu baseline (restated reference rollout, bounded sample) ...")
            cpu = cpu_baseline_rollout(model, prompts)
            # the sample's two rates applied to this run's token mix (its prompt and
            # generated token counts): an estimate of the CPU path on the whole cfg4
            # job, reported beside the measured sample rate, never as `value`
            gen, ptok = ro["tokens"] // steps, sum(len(p) for p in prompts)
            cpu["cfg4_mix_estimate_tok_s"] = gen / (ptok / cpu["prefill_tok_s"] + gen / cpu["decode_tok_s"])
            log(f"[bench] cpu: {cpu['sample']}; cfg4 mix estimate {cpu['cfg4_mix_estimate_tok_s']:.0f} tok/s")
        c5 = None
        if not a.no_cfg5:
            del model
            torch.cuda.empty_cache()
            r5 = rollout_cfg5(1, 1, dev)
            run5 = r5["runs"][-1]
            c5 = {"tokens_per_s": r5["value"], "generated_tokens": r5["tokens"], "prompt_tokens": r5["prompt_tokens"],
                  "decode_steps": run5["decode_steps"], "prefill_s": run5["prefill_s"], "decode_s": run5["decode_s"],
                  "workload": "RWKV7-7.2B (L=32, C=4096, H=64) bf16, 128 prompts x 2048 tokens, chunk 256, "
                              "temp 1.0, top_p 0.95, max 1024 new, geometric(600) stops, 128 slots; 1 timed rollout "
                              "after 1 warm-up"}
            log(f"[bench] cfg5: {r5['value']:.0f} tokens/s")
        out = {
            "metric": METRIC, "value": ro["value"], "unit": "tokens/s", "n_gpus": 1, "steps": steps,
            "warmup": warmup, "ms_per_step": ro["ms_per_step"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16 weights/activations, fp32 WKV state and element-wise",
            "data": "synthetic (random prompts, seeded dense random-init weights)",
            "config": {"workload": "cfg4 GRPO rollout: RWKV7-1.5B, 64 prompts U(256,2048) x 8 = 512 seqs, "
                                   "temp 1.0, top_p 0.95, max 512 new, geometric(300) stops, 256 slots",
                       "global_batch": 512, "seq_len": 2048 + 512, "parallelism": "none (1 GPU)",
                       "generated_tokens": ro["tokens"] // steps, "prompt_tokens": sum(len(p) for p in prompts),
                       "decode_steps": ro["runs"][-1]["decode_steps"],
                       "prefill_s": ro["runs"][-1]["prefill_s"], "decode_s": ro["runs"][-1]["decode_s"]},
            "roofline": {"bound": "hbm", "achieved": gm["GBs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gm["frac"], "traffic": gemm_pmc_traffic(), "kernel": gm["kernel"],
                         "M": gm["M"], "us_per_launch": gm["us_per_layer"] / 5,
                         "algorithmic_bytes": gm["weight_bytes_per_layer"] / 5},
            "roofline_tmix": {"bound": "hbm", "achieved": tm["GBs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                              "frac": tm["frac"], "traffic": pmc_traffic(), "kernel": tm["kernel"],
                              "us_per_launch": tm["us_per_launch"], "algorithmic_bytes": tm["bytes_per_launch"]},
            "roofline_rollout": rr,
            "cfg5_rollout": c5,
            "wkv7_decode_cfg2": {"GBs": wk["GBs"], "frac": wk["frac"], "us_per_step": wk["us_per_step"]},
            "wkv7_prefill_cfg3": dict({k: pf[k] for k in ("us_per_launch", "tokens_per_s", "algorithmic_TFLOPs",
                                                          "mfma_bf16_TFLOPs", "mfma_frac", "GBs", "hbm_frac",
                                                          "speedup_vs_token_serial")},
                                      algorithmic_frac=pf["algorithmic_TFLOPs"] / PEAK_BF16_TFLOPS),
            "cpu_baseline": cpu,
        }
    elif a.workload == "scheduler":
        steps = 2 if a.steps is None else a.steps
        warmup = 1 if a.warmup is None else a.warmup
        sc = scheduler_rollout(steps, warmup, dev)
        run = sc["runs"][-1]
        out = {
            "metric": METRIC, "value": sc["value"], "unit": "tokens/s", "n_gpus": 1, "steps": steps,
            "warmup": warmup, "ms_per_step": sc["ms_per_step"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16 weights/activations, fp32 WKV state and element-wise",
            "data": "synthetic (random prompts, seeded dense random-init weights)",
            "config": {"workload": "cfg4's 512 sequences (64 prompts U(256,2048) x 8 copies, geometric(300) stops, "
                                   "max 512 new) through BatchGenerator with 256 slots: each copy's prompt "
                                   "prefilled in its own slot on admission (16,384 tokens per forward, chunks of "
                                   "2,048), temp 1.0, top_p 0.95",
                       "global_batch": 512, "seq_len": 2048 + 512, "parallelism": "none (1 GPU)",
                       "generated_tokens": sc["tokens"] // steps, "prompt_tokens": sc["prompt_tokens"],
                       "decode_steps": run["decode_steps"], "prefill_passes": run["prefill_passes"],
                       "prefill_host_s": run["prefill_host_s"], "total_s": run["total_s"]},
            "roofline": None,
            "cpu_baseline": None,
        }
    elif a.workload == "cfg5":
        steps = 1 if a.steps is None else a.steps
        warmup = 1 if a.warmup is None else a.warmup
        ro = rollout_cfg5(steps, warmup, dev)
        log("[bench] fused decode time-mix kernel at the cfg5 shape (roofline) ...")
        tm = tmix_decode_leg(dev, S=128, H=64, L=32)
        log(f"[bench] tmix_decode cfg5 shape: {tm['us_per_launch']:.2f} us/launch, {tm['GBs']:.0f} GB/s")
        run = ro["runs"][-1]
        out = {
            "metric": METRIC, "value": ro["value"], "unit": "tokens/s", "n_gpus": 1, "steps": steps,
            "warmup": warmup, "ms_per_step": ro["ms_per_step"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16 weights/activations, fp32 WKV state and element-wise",
            "data": "synthetic (random prompts, seeded dense random-init weights)",
            "config": {"workload": "cfg5 rollout: RWKV7-7.2B (L=32, C=4096, H=64), 128 prompts x 2048 tokens, "
                                   "chunked prefill (chunk 256), temp 1.0, top_p 0.95, max 1024 new, "
                                   "geometric(600) stops, 128 slots",
                       "global_batch": 128, "seq_len": 2048 + 1024, "parallelism": "none (1 GPU)",
                       "generated_tokens": ro["tokens"] // steps, "prompt_tokens": ro["prompt_tokens"],
                       "decode_steps": run["decode_steps"], "prefill_s": run["prefill_s"],
                       "decode_s": run["decode_s"]},
            "roofline": {"bound": "hbm", "achieved": tm["GBs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": tm["frac"], "traffic": None, "kernel": tm["kernel"] + " at 128 slots, H=64",
                         "us_per_launch": tm["us_per_launch"], "algorithmic_bytes": tm["bytes_per_launch"]},
            "cpu_baseline": None,
        }
    elif a.workload == "logprob":
        steps = 2 if a.steps is None else a.steps
        warmup = 1 if a.warmup is None else a.warmup
        model, lp = logprob_recompute(steps, warmup, dev)
        cpu = None
        if not a.no_cpu_baseline:
            log("[bench] cpu baseline (restated reference recompute, one sequence) ...")
            cpu = cpu_baseline_logprob(model)
            log(f"[bench] cpu: {cpu['sample']}")
        out = {
            "metric": METRIC, "value": lp["value"], "unit": "forward tokens/s", "n_gpus": 1, "steps": steps,
            "warmup": warmup, "ms_per_step": lp["seconds"] * 1e3, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16 weights/activations, fp32 WKV state and log-softmax",
            "data": "synthetic (random ids, seeded dense random-init weights)",
            "config": {"workload": "GRPO log-prob recompute after a cfg4 rollout: RWKV7-1.5B, 512 seqs "
                                   "(64 prompts x 8) of 1024 prompt + 512 completion tokens, padded to "
                                   f"{lp['T']}", "global_batch": 512, "seq_len": lp["T"],
                       "parallelism": "none (1 GPU)", "completion_tokens": lp["completion_tokens"]},
            "roofline": {"bound": "mfma", "achieved": lp["gemm_TFLOPs"], "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": lp["gemm_TFLOPs"] / PEAK_BF16_TFLOPS, "traffic": None,
                         "kernel": "whole recompute (block GEMMs at every position + head at the completion "
                                   "positions), per second of wall time", "flops_per_step": lp["flops"]},
            "cpu_baseline": cpu,
        }
    elif a.workload == "train":
        steps = 5 if a.steps is None else a.steps
        warmup = 1 if a.warmup is None else a.warmup
        tr = train_leg(dev, steps, warmup)
        log(f"[bench] train op: fwd {tr['fwd_ms']:.2f} ms ({tr['fwd_GBs']:.0f} GB/s), bwd {tr['bwd_ms']:.2f} ms "
            f"({tr['bwd_GBs']:.0f} GB/s), {tr['tokens_per_s']:.0f} tokens/s")
        cpu = None if a.no_cpu_baseline else cpu_baseline_train()
        out = {
            "metric": METRIC, "value": tr["tokens_per_s"], "unit": "tokens/s (WKV7 forward + backward, one layer)",
            "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": tr["fwd_ms"] + tr["bwd_ms"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16 I/O, fp32 state and checkpoints", "data": "synthetic",
            "config": {"workload": f"WKV7 training operator, B={tr['B']} x T={tr['T']}, H={tr['H']}, N=64",
                       "fwd_ms": tr["fwd_ms"], "bwd_ms": tr["bwd_ms"], "fwd_GBs": tr["fwd_GBs"]},
            "roofline": {"bound": "hbm", "achieved": tr["bwd_GBs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": tr["bwd_GBs"] / PEAK_HBM_GBS, "traffic": None, "kernel": tr["kernels"]},
            "cpu_baseline": cpu,
        }
    elif a.workload == "gemm":
        # the decode step's projections alone (for kernel-trace / PMC runs) at --rows
        # rows over the 1.5B model's 24 layers, then a plain copy of known size
        from rwkvtune_amd.model import build_model, config_from_preset
        reps = 10 if a.steps is None else a.steps
        model = build_model(config_from_preset("rwkv7-1.5b"), dtype=torch.bfloat16, device=dev, seed=1234)
        gm = gemm_decode_leg(model, dev, M=a.rows, reps=reps)
        ref = copy_reference(dev)
        out = {
            "metric": METRIC, "value": gm["GBs"], "unit": "GB/s of packed weights", "n_gpus": 1, "steps": reps,
            "warmup": 1, "ms_per_step": gm["us_per_layer"] * 24 / 1e3, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16 in, fp32 accumulate", "data": "synthetic",
            "config": {"workload": f"decode projections of RWKV7-1.5B (5 grouped GEMM launches per layer, 24 "
                                   f"layers in turn) at M={a.rows} rows", "copy_reference_bytes": ref},
            "roofline": {"bound": "hbm", "achieved": gm["GBs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gm["frac"], "traffic": gemm_pmc_traffic() if a.rows == 256 else None,
                         "kernel": gm["kernel"], "M": a.rows, "us_per_launch": gm["us_per_layer"] / 5,
                         "algorithmic_bytes": gm["weight_bytes_per_layer"] / 5},
            "cpu_baseline": None,
        }
    elif a.workload == "sampler":
        # one sampling step at --rows rows: LM head + sampler (for kernel-trace runs)
        reps = 200 if a.steps is None else a.steps
        hs = head_sampler_leg(dev, M=a.rows, reps=reps, C=a.embd)
        copy_reference(dev)  # scales the PMC byte counters of the head profile
        own_head = hs["head_kernel"] and a.rows == 128 and a.embd == 2048
        out = {
            "metric": METRIC, "value": hs["tokens_per_s"], "unit": "sampled tokens/s", "n_gpus": 1, "steps": reps,
            "warmup": 2, "ms_per_step": hs["step_us"] / 1e3, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16 head and logits, fp32 sampling", "data": "synthetic",
            "config": {"workload": f"sampling step at {a.rows} rows: LM head [{a.rows}, {a.embd}] x "
                                   f"[65536, {a.embd}]^T ({'head_logits_kernel' if hs['head_kernel'] else 'hipBLASLt'})"
                                   " + sampler (RULE_BATCH, temperature 1, top_p 0.95)"},
            "roofline": {"bound": "hbm", "achieved": hs["head_GBs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": hs["head_GBs"] / PEAK_HBM_GBS,
                         "traffic": head_pmc_traffic() if own_head else None,
                         "kernel": "head_logits_kernel" if hs["head_kernel"] else "LM head GEMM (hipBLASLt)",
                         "us_per_launch": hs["head_us"], "algorithmic_bytes": 65536 * a.embd * 2},
            "head_us": hs["head_us"], "head_lib_us": hs["head_lib_us"], "sampler_us": hs["sampler_us"],
            "step_us": hs["step_us"],
            "draws_valid": hs["valid"], "cpu_baseline": None,
        }
    elif a.workload == "tmix":
        # the roofline kernel alone (for kernel-trace / PMC runs), then a plain copy of
        # known size that scales the PMC byte counters
        steps = 480 if a.steps is None else a.steps
        warmup = 48 if a.warmup is None else a.warmup
        tm = tmix_decode_leg(dev, iters=steps)
        ref = copy_reference(dev)
        out = {
            "metric": METRIC, "value": tm["GBs"], "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
            "ms_per_step": tm["us_per_launch"] / 1e3, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16 I/O, fp32 state and element-wise", "data": "synthetic",
            "config": {"workload": "fused decode time-mix (tmix_decode_kernel) at the cfg4 decode shape: 256 rows, "
                                   "H=32, 24 rotating layer pools", "copy_reference_bytes": ref},
            "roofline": {"bound": "hbm", "achieved": tm["GBs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": tm["frac"], "traffic": pmc_traffic(), "kernel": tm["kernel"],
                         "us_per_launch": tm["us_per_launch"], "algorithmic_bytes": tm["bytes_per_launch"]},
            "cpu_baseline": None,
        }
    elif a.workload == "prefill":
        steps = 20 if a.steps is None else a.steps
        warmup = 3 if a.warmup is None else a.warmup
        pf = prefill_leg(dev, iters=steps)
        cpu = None if a.no_cpu_baseline else cpu_baseline_prefill()
        out = {
            "metric": METRIC, "value": pf["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": steps,
            "warmup": warmup, "ms_per_step": pf["us_per_launch"] / 1e3, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16 I/O, bf16 MFMA (hi/lo operand split), fp32 state",
            "data": "synthetic",
            "config": {"workload": f"cfg3 WKV7 ragged chunked prefill: 64 prompts U(64,2048) = {pf['tokens']} "
                                   "tokens, H=32, N=64, zero initial state"},
            "roofline": {"bound": "mfma", "achieved": pf["mfma_bf16_TFLOPs"], "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": pf["mfma_frac"], "traffic": None, "kernel": pf["kernel"],
                         "algorithmic_TFLOPs": pf["algorithmic_TFLOPs"], "hbm_GBs": pf["GBs"],
                         "hbm_frac": pf["hbm_frac"]},
            "token_serial_us": pf["token_serial_us"], "speedup_vs_token_serial": pf["speedup_vs_token_serial"],
            "cpu_baseline": cpu,
        }
    else:
        steps = 1000 if a.steps is None else a.steps
        warmup = 50 if a.warmup is None else a.warmup
        wk = wkv_decode_leg(dev, iters=steps)
        tm = tmix_decode_leg(dev)
        cpu = None if a.no_cpu_baseline else cpu_baseline_decode()
        out = {
            "metric": METRIC, "value": wk["GBs"], "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
            "ms_per_step": wk["us_per_step"] / 1e3, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16 I/O, fp32 state", "data": "synthetic",
            "config": {"workload": "cfg2 WKV7 decode step, B=256 slots, H=32, N=64, 8 rotating state pools"},
            "roofline": {"bound": "hbm", "achieved": wk["GBs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": wk["frac"], "traffic": None, "kernel": wk["kernel"]},
            "tmix_decode": {"GBs": tm["GBs"], "frac": tm["frac"], "us_per_launch": tm["us_per_launch"]},
            "cpu_baseline": cpu,
        }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
