"""GPU parity of the WKV7 decode / token-serial kernels against the fp64 oracle.

Tolerances (stated once, used everywhere below):
  y      bf16/fp16 I/O: ||y - round(y_ref)|| / ||round(y_ref)|| <= 1e-3 over the whole
         output, where round() is the I/O type's rounding of the fp64 oracle (the
         reference kernel also returns y in the I/O type, wkv7s.cu:49); and every
         element is a faithful rounding up to fp32 accumulation error:
         |y - y_ref| <= 1 ulp of the I/O type at y_ref + 1e-5 * rms(y_ref).
         (A per-(slot, head) norm is not used for bf16: one legitimate
         rounding flip of a head's largest element already costs ~1e-3 of that head.)
         fp32 I/O: per (slot, head) ||y - y_ref|| / ||y_ref|| <= 1e-5.
  state  fp32: per (slot, head) ||S - S_ref|| / ||S_ref|| <= 1e-4.
Chunked prefill with bf16/fp16 I/O multiplies operands split into two bf16 parts
(hi + lo, relative error per product ~2^-16), so its per-element bound is
|y - y_ref| <= 1 ulp + 2e-4 * rms(y_ref) (CHUNK16_ATOL); the norm-wise 1e-3 bound
on y and the 1e-4 state bound are the same as above.  Chunked prefill with fp32
I/O uses a three-part split (~2^-24 per product) and keeps the fp32 bounds.
"""

import pytest
import torch

from oracle.wkv7 import wkv7_ragged, wkv7_rowwise
from rwkvtune_amd import operators as ops
from rwkvtune_amd.workloads import cu_seqlens_of, ragged_lengths, wkv_inputs, wkv_state

pytestmark = pytest.mark.gpu

N = 64
Y_TOL = {torch.bfloat16: 1e-3, torch.float16: 1e-3, torch.float32: 1e-5}
S_TOL = 1e-4


def per_head_rel(x, ref, H):
    """max over (row, head) of ||x - ref|| / ||ref|| on [..., H*N] tensors."""
    x = x.double().reshape(-1, H, N)
    ref = ref.double().reshape(-1, H, N)
    num = (x - ref).norm(dim=-1)
    den = ref.norm(dim=-1).clamp_min(1e-30)
    return float((num / den).max())


def state_rel(S, ref):
    S = S.double().reshape(-1, N * N)
    ref = ref.double().reshape(-1, N * N)
    return float(((S - ref).norm(dim=-1) / ref.norm(dim=-1).clamp_min(1e-30)).max())


MANT_BITS = {torch.bfloat16: 7, torch.float16: 10}


def ulp(x, dtype):
    e = torch.floor(torch.log2(x.abs().clamp_min(1e-30)))
    if dtype == torch.float16:
        e = e.clamp_min(-14)
    return torch.pow(2.0, e - MANT_BITS[dtype])


CHUNK16_ATOL = 2e-4


def check_y(y_gpu, y_ref64, H, dtype, atol_rms=1e-5):
    y = y_gpu.cpu().double()
    if dtype == torch.float32:
        rel = per_head_rel(y, y_ref64, H)
        assert rel <= Y_TOL[dtype], f"y per-head rel err {rel:.3e}"
        return rel
    ref = y_ref64.to(dtype).double()
    rel = float((y - ref).norm() / ref.norm())
    assert rel <= Y_TOL[dtype], f"y rel err {rel:.3e}"
    atol = atol_rms * float(y_ref64.pow(2).mean().sqrt())
    bad = (y - y_ref64).abs() > ulp(y_ref64, dtype) * 1.0001 + atol
    assert not bool(bad.any()), f"{int(bad.sum())} elements not faithfully rounded"
    return rel


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_decode_cfg2_shape(gpu_device, dtype):
    """Isolated decode step at the benchmark shape: B=256 slots, H=32."""
    B, H = 256, 32
    print(f"[case] decode B={B} H={H} dtype={dtype}", flush=True)
    inp = wkv_inputs((B,), H, N, seed=100, dtype=dtype)
    S0 = wkv_state(B, H, N, seed=101)
    y_ref, S_ref = wkv7_rowwise(*(t.unsqueeze(1) for t in inp.as_tuple()), N, S0)
    pool = S0.to(gpu_device)
    g = inp.to(gpu_device)
    y = ops.wkv7_decode(pool, None, *g.as_tuple())
    torch.cuda.synchronize()
    check_y(y, y_ref[:, 0], H, dtype)
    assert state_rel(pool.cpu(), S_ref) <= S_TOL


def test_decode_slot_table_and_skip(gpu_device):
    """Rows address pool slots through slot_idx; negative slots are skipped."""
    B, H, S = 6, 4, 9
    print("[case] decode slot table", flush=True)
    inp = wkv_inputs((B,), H, N, seed=102)
    pool0 = wkv_state(S, H, N, seed=103)
    slots = [7, 0, -1, 3, 8, 2]
    pool = pool0.to(gpu_device)
    sidx = torch.tensor(slots, dtype=torch.int32, device=gpu_device)
    y = torch.full((B, H * N), 7.0, dtype=torch.bfloat16, device=gpu_device)
    ops.wkv7_decode(pool, sidx, *inp.to(gpu_device).as_tuple(), y=y)
    torch.cuda.synchronize()
    pool = pool.cpu()
    y = y.cpu()
    for i, s in enumerate(slots):
        if s < 0:
            assert torch.all(y[i] == 7.0)
            continue
        yr, Sr = wkv7_rowwise(*(t[i:i + 1, None] for t in inp.as_tuple()), N, pool0[s:s + 1])
        check_y(y[i:i + 1], yr[:, 0], H, torch.bfloat16)
        assert state_rel(pool[s:s + 1], Sr) <= S_TOL
    used = {s for s in slots if s >= 0}
    for s in range(S):
        if s not in used:
            assert torch.equal(pool[s], pool0[s])


def test_repeated_decode_steps_long(gpu_device):
    """1000 consecutive decode steps on a small batch track the fp64 oracle."""
    B, H, T = 2, 2, 1000
    print("[case] 1000 decode steps", flush=True)
    inp = wkv_inputs((B, T), H, N, seed=104)
    S0 = wkv_state(B, H, N, seed=105)
    y_ref, S_ref = wkv7_rowwise(*inp.as_tuple(), N, S0)
    pool = S0.to(gpu_device)
    g = inp.to(gpu_device)
    ys = []
    for t in range(T):
        ys.append(ops.wkv7_decode(pool, None, *(x[:, t] for x in g.as_tuple())))
    y = torch.stack(ys, 1)
    torch.cuda.synchronize()
    check_y(y, y_ref, H, torch.bfloat16)
    assert state_rel(pool.cpu(), S_ref) <= S_TOL


def test_cfg2_1000_steps_linearity(gpu_device):
    """At the full cfg2 shape, 1000 steps: the map (S0, v) -> (S_T, y) is linear
    for fixed r, w, k, a, b, so scaling S0 and v by 2^-3 scales every output by
    exactly 2^-3 (bit-exact in fp32 arithmetic; y compared before bf16 rounding
    via fp32 I/O)."""
    B, H, T = 256, 32, 1000
    print("[case] cfg2 1000 steps linearity", flush=True)
    g = wkv_inputs((B,), H, N, seed=106, dtype=torch.float32).to(gpu_device)
    S0 = wkv_state(B, H, N, seed=107).to(gpu_device)
    pa = S0.clone()
    pb = (S0 * 0.125).contiguous()
    vb = g.v * 0.125
    for _ in range(T):
        ya = ops.wkv7_decode(pa, None, g.r, g.w, g.k, g.v, g.a, g.b)
        yb = ops.wkv7_decode(pb, None, g.r, g.w, g.k, vb, g.a, g.b)
    torch.cuda.synchronize()
    assert torch.isfinite(pa).all()
    assert torch.equal(pa * 0.125, pb)
    assert torch.equal(ya * 0.125, yb)


@pytest.mark.parametrize("chunk_len", [1, 0])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_ragged_prefill(gpu_device, dtype, chunk_len):
    """Ragged prompts (empty, single-token, partial and whole 32-token chunks)
    into chosen slots: token-serial (chunk_len=1) and chunked (chunk_len=0)."""
    H = 4
    lens = [1, 0, 37, 5, 64, 130]
    print(f"[case] ragged prefill {lens} dtype={dtype} chunk_len={chunk_len}", flush=True)
    cu = cu_seqlens_of(lens)
    inp = wkv_inputs((cu[-1],), H, N, seed=108, dtype=dtype)
    pool0 = wkv_state(8, H, N, seed=109)
    slots = [5, 1, 0, 7, 2, 6]
    y_ref, fin = wkv7_ragged(*inp.as_tuple(), cu, states=pool0[slots])
    pool = pool0.to(gpu_device)
    y = ops.wkv7_prefill(pool, torch.tensor(slots, dtype=torch.int32, device=gpu_device),
                         torch.tensor(cu, dtype=torch.int32, device=gpu_device),
                         *inp.to(gpu_device).as_tuple(), chunk_len=chunk_len)
    torch.cuda.synchronize()
    check_y(y, y_ref, H, dtype, atol_rms=CHUNK16_ATOL if chunk_len != 1 else 1e-5)
    assert state_rel(pool.cpu()[slots], fin) <= S_TOL
    assert torch.equal(pool.cpu()[[3, 4]], pool0[[3, 4]])


def decay_regime_inputs(seed):
    """fp32 inputs of 4 sequences x 4 heads whose decays cover the chunked
    kernel's regimes: per-token log-decay -exp(w) of
      head 0: ~-1e-9 (no decay: D = 1 to fp32),
      head 1: -1.2 (just above the matrix form's floor of -1.25: operands span e^+-38),
      head 2: -2.7 (below the floor: the exact serial fallback),
      head 3: alternating by 32-token chunk between -0.3 and -2.7 (both paths
              in one sequence, state carried between them),
    plus the trained-model range (w <= -0.5) on sequence 3."""
    H = 4
    lens = [100, 64, 33, 96]
    cu = cu_seqlens_of(lens)
    inp = wkv_inputs((cu[-1],), H, N, seed=seed, dtype=torch.float32)
    w = inp.w.view(-1, H, N)
    w[:, 0] = -20.0
    w[:, 1] = float(torch.log(torch.tensor(1.2)))
    w[:, 2] = 1.0
    for si, (tb, te) in enumerate(zip(cu[:-1], cu[1:])):
        for t in range(tb, te):
            w[t, 3] = -1.2 if ((t - tb) // 32) % 2 == 0 else 1.0
    tb, te = cu[3], cu[4]
    w[tb:te] = w[tb:te].clamp_max(-0.5)
    return inp, lens, cu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_chunked_prefill_decay_regimes(gpu_device, dtype):
    H = 4
    print(f"[case] chunked prefill decay regimes {dtype}", flush=True)
    inp, lens, cu = decay_regime_inputs(112)
    inp = type(inp)(*(t.to(dtype) for t in inp.as_tuple()))
    pool0 = wkv_state(len(lens), H, N, seed=113)
    y_ref, fin = wkv7_ragged(*inp.as_tuple(), cu, states=pool0)
    pool = pool0.to(gpu_device)
    y = ops.wkv7_prefill(pool, None, torch.tensor(cu, dtype=torch.int32, device=gpu_device),
                         *inp.to(gpu_device).as_tuple(), chunk_len=32)
    torch.cuda.synchronize()
    check_y(y, y_ref, H, dtype, atol_rms=CHUNK16_ATOL)
    assert state_rel(pool.cpu(), fin) <= S_TOL


@pytest.mark.parametrize("chunk_len", [16, 32, 64])
def test_chunk_len_values_same_result(gpu_device, chunk_len):
    """chunk_len 16/32/64 name the caller's chunking; the result is the recurrence's."""
    H = 2
    lens = [70, 3]
    cu = cu_seqlens_of(lens)
    print(f"[case] chunk_len={chunk_len}", flush=True)
    inp = wkv_inputs((cu[-1],), H, N, seed=114, dtype=torch.float32).to(gpu_device)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=gpu_device)
    p0 = torch.zeros(2, H, N, N, device=gpu_device)
    p1 = p0.clone()
    y0 = ops.wkv7_prefill(p0, None, cu_d, *inp.as_tuple(), chunk_len=0)
    y1 = ops.wkv7_prefill(p1, None, cu_d, *inp.as_tuple(), chunk_len=chunk_len)
    assert torch.equal(y0, y1) and torch.equal(p0, p1)
    with pytest.raises(ValueError):
        ops.wkv7_prefill(p1, None, cu_d, *inp.as_tuple(), chunk_len=48)


def test_chunked_prefill_cfg3_shape(gpu_device):
    """cfg3: 64 prompts with lengths ~U(64, 2048), H=32, bf16 inputs drawn as in
    cfg2, zero initial state.  All 64 sequences: chunked equals the token-serial
    kernel (y within 1e-3 relative as bf16 outputs, state per (seq, head) within
    1e-4); the shortest, a middle and the longest sequence against the fp64 C
    oracle at the stated tolerances."""
    from oracle import cref
    H = 32
    lens = ragged_lengths(64, 64, 2048, seed=3)
    cu = cu_seqlens_of(lens)
    print(f"[case] cfg3 chunked prefill total={cu[-1]}", flush=True)
    inp = wkv_inputs((cu[-1],), H, N, seed=115)
    g = inp.to(gpu_device)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=gpu_device)
    pc = torch.zeros(64, H, N, N, device=gpu_device)
    ps = torch.zeros(64, H, N, N, device=gpu_device)
    yc = ops.wkv7_prefill(pc, None, cu_d, *g.as_tuple(), chunk_len=64)
    ys = ops.wkv7_prefill(ps, None, cu_d, *g.as_tuple(), chunk_len=1)
    torch.cuda.synchronize()
    e = float((yc.double() - ys.double()).norm() / ys.double().norm())
    assert e <= 1e-3, f"chunked vs serial y rel err {e:.3e}"
    assert state_rel(pc.cpu(), ps.cpu()) <= S_TOL
    order = sorted(range(64), key=lambda i: lens[i])
    for si in (order[0], order[32], order[-1]):
        tb, te = cu[si], cu[si + 1]
        y_ref, S_ref = cref.wkv7_ref_f64(*(t[tb:te][None] for t in inp.as_tuple()))
        check_y(yc[tb:te].cpu(), y_ref[0], H, torch.bfloat16, atol_rms=CHUNK16_ATOL)
        assert state_rel(pc[si:si + 1].cpu(), S_ref) <= S_TOL


def test_uniform_batch_prefill_operator(gpu_device):
    """rwkv7_wkv on [B, T, C] with T > 1 runs the chunked kernel on uniform
    lengths; each batch row equals its own fp64 recurrence."""
    B, H, T = 3, 2, 70
    print("[case] uniform [B,T,C] chunked", flush=True)
    inp = wkv_inputs((B, T), H, N, seed=116)
    S0 = wkv_state(B, H, N, seed=117)
    y_ref, S_ref = wkv7_rowwise(*inp.as_tuple(), N, S0)
    st = S0.to(gpu_device)
    y = ops.rwkv7_wkv(*inp.to(gpu_device).as_tuple(), head_size=64, state=st)
    torch.cuda.synchronize()
    check_y(y, y_ref, H, torch.bfloat16, atol_rms=CHUNK16_ATOL)
    assert state_rel(st.cpu(), S_ref) <= S_TOL


def test_reference_operator_contract(gpu_device):
    """load_wkv_operator('cuda', for_inference=True) behaves like RUN_CUDA_RWKV7S."""
    op = ops.load_wkv_operator(device="cuda", for_inference=True, head_size=64)
    assert op is ops.load_wkv7_operator("cuda", True, 64)
    H, T = 2, 9
    inp = wkv_inputs((T,), H, N, seed=110).to(gpu_device)
    with pytest.raises(ValueError):
        op(*inp.as_tuple())
    with pytest.raises(RuntimeError):
        op(*(t[None, None] for t in inp.as_tuple()), state=torch.zeros(1, H, N, N, device=gpu_device))
    with pytest.raises(RuntimeError):
        op(*(t.to(torch.float64) for t in inp.as_tuple()), state=torch.zeros(1, H, N, N, device=gpu_device))
    S0 = wkv_state(1, H, N, seed=111)
    state = S0[0].to(gpu_device).contiguous()
    y, st = op(*inp.as_tuple(), state=state, return_state=True)
    assert st is state and y.shape == (T, H * N) and y.dtype == torch.bfloat16
    y_ref, S_ref = wkv7_rowwise(*(t.cpu() for t in inp.as_tuple()), N, S0[0])
    check_y(y, y_ref, H, torch.bfloat16, atol_rms=CHUNK16_ATOL)
    assert state_rel(state.cpu(), S_ref) <= S_TOL
    # batched form through rwkv7_wkv
    st2 = S0.to(gpu_device)
    y2 = ops.rwkv7_wkv(*(t[None] for t in inp.as_tuple()), head_size=64, state=st2)
    check_y(y2[0], y_ref, H, torch.bfloat16, atol_rms=CHUNK16_ATOL)


def test_chunked_prefill_fp16_and_misaligned_inputs(gpu_device):
    """fp16 I/O through the 16-bit chunked kernel; input views whose data pointers
    are not 8-byte aligned are copied by the operator before the launch (the C ABI
    rejects them) and give the same result."""
    H = 2
    lens = [45, 70]
    cu = cu_seqlens_of(lens)
    print("[case] chunked fp16 + misaligned", flush=True)
    for dtype, shift in ((torch.float16, 0), (torch.bfloat16, 1)):
        inp = wkv_inputs((cu[-1],), H, N, seed=118, dtype=dtype)
        y_ref, fin = wkv7_ragged(*inp.as_tuple(), cu)
        g = []
        for t in inp.as_tuple():
            buf = torch.empty(t.numel() + 8, dtype=dtype, device=gpu_device)
            view = buf[shift:shift + t.numel()].view(t.shape)   # shift=1: 2-byte aligned only
            view.copy_(t.to(gpu_device))
            g.append(view)
        pool = torch.zeros(2, H, N, N, device=gpu_device)
        y = ops.wkv7_prefill(pool, None, torch.tensor(cu, dtype=torch.int32, device=gpu_device), *g)
        torch.cuda.synchronize()
        check_y(y, y_ref, H, dtype, atol_rms=CHUNK16_ATOL)
        assert state_rel(pool.cpu(), fin) <= S_TOL
