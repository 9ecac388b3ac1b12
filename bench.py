#!/usr/bin/env python3
"""Benchmark of the WKV7 decode / prefill / rollout hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload rollout|decode]

Prints ONE JSON line (see the keys at the end of main()).  One GPU only:
``--gpus N`` with N > 1 exits with a message.

Workloads
---------
decode   isolated WKV7 decode step: B=256 slots, H=32, N=64, fp32 state, bf16 I/O,
         a "step" is one kernel launch over all 8192 (slot, head) units.
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

PEAK_HBM_GBS = 8000.0          # MI355X datasheet HBM3E bandwidth
METRIC = "rollout tokens/s (RWKV7-1.5B, 512 seqs); WKV7 decode HBM GB/s vs peak"
N = 64
# algorithmic bytes of one decode (slot, head) unit: fp32 state read + write,
# six bf16 inputs of N, bf16 output of N
DECODE_BYTES_PER_UNIT = 2 * N * N * 4 + 6 * N * 2 + N * 2


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def decode_cfg2(steps: int, warmup: int, dev):
    """Time `steps` decode launches at B=256, H=32 with HIP events on the launch stream."""
    from rwkvtune_amd import operators as ops
    from rwkvtune_amd.workloads import wkv_inputs, wkv_state

    B, H = 256, 32
    inp = wkv_inputs((B,), H, N, seed=1000).to(dev)
    pool = wkv_state(B, H, N, seed=1001).to(dev)
    y = torch.empty_like(inp.r)
    args = inp.as_tuple()
    for _ in range(warmup):
        ops.wkv7_decode(pool, None, *args, y=y)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        ops.wkv7_decode(pool, None, *args, y=y)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    us = ms * 1e3 / steps
    units = B * H
    gbs = units * DECODE_BYTES_PER_UNIT / (us * 1e-6) / 1e9
    return {"B": B, "H": H, "us_per_step": us, "bytes_per_step": units * DECODE_BYTES_PER_UNIT,
            "achieved_GBs": gbs, "frac": gbs / PEAK_HBM_GBS, "steps": steps}


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
    gbs = B * H * DECODE_BYTES_PER_UNIT / dt / 1e9
    return {"value": gbs, "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"one cfg2 decode step (B=256,H=32) through the restated wkv_cpu.py path, "
                      f"fp32, mean of {reps}; {dt * 1e3:.1f} ms/step"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="decode", choices=["decode"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {a.gpus}); the rollout shards "
              "by sequence with no cross-GPU exchange, see DESIGN.md", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    from rwkvtune_amd import _lib
    _lib.load()

    log("[bench] decode cfg2 ...")
    dec = decode_cfg2(a.steps, a.warmup, dev)
    log(f"[bench] decode: {dec['us_per_step']:.2f} us/step, {dec['achieved_GBs']:.0f} GB/s")
    cpu = None
    if not a.no_cpu_baseline:
        log("[bench] cpu baseline ...")
        cpu = cpu_baseline_decode()
    out = {
        "metric": METRIC,
        "value": dec["achieved_GBs"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": dec["us_per_step"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 I/O, fp32 state",
        "data": "synthetic",
        "config": {"workload": "wkv7 decode step, B=256 slots, H=32, N=64 (cfg2)"},
        "roofline": {"bound": "hbm", "achieved": dec["achieved_GBs"], "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": dec["frac"], "traffic": None},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
