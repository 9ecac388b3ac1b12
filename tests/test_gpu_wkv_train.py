"""WKV7 training operator (rwkv7_wkv_train_forward / _backward and the Python
WindBackstepping / infctx wrappers) against the restated reference algorithm
(oracle/wkv7_train.py, float64, itself pinned to torch autograd).

Tolerances, written per test:
* float32 I/O: the forward and the gradients within 1e-4 of each tensor's largest
  magnitude for decays >= 0.87; for decays down to 0.55 the backward's step-back
  (division by the decay over up to 15 tokens, as the reference) amplifies float32
  rounding, so 2e-3.
* bf16 I/O (the standard training op): inputs rounded to bf16 first; y within one
  bf16 ulp + 2e-3 of max|y|, gradients within 2e-2 of their largest magnitude
  (bf16 output rounding of sums over 64 terms and the step-back).
"""

import pytest
import torch

from oracle import wkv7 as ow
from oracle import wkv7_train as otr
from rwkvtune_amd import operators as ops

pytestmark = pytest.mark.gpu


def inputs(B, T, H, lo, hi, seed, N=64):
    g = torch.Generator().manual_seed(seed)
    shp = (B, T, H, N)
    r = torch.randn(shp, generator=g)
    k = torch.randn(shp, generator=g) * 0.5
    v = torch.randn(shp, generator=g)
    w = torch.rand(shp, generator=g) * (hi - lo) + lo         # raw: decay exp(-exp(w))
    kk = torch.nn.functional.normalize(torch.randn(shp, generator=g), dim=-1)
    iclr = torch.rand(shp, generator=g)
    return [r, w, k, v, -kk, kk * iclr]


def close(got, ref, frac):
    ref = ref.double().cpu()
    return float((got.double().cpu() - ref).abs().max()) <= frac * float(ref.abs().max()) + 1e-12


def y_close(y, ref, dtype):
    """A 16-bit output: within one ulp of its type + 2e-3 of the largest magnitude."""
    ref = ref.double().cpu()
    err = (y.double().cpu() - ref).abs()
    return bool((err <= torch.finfo(dtype).eps * ref.abs() + 2e-3 * float(ref.abs().max())).all())


@pytest.mark.parametrize("T,with_state,lo,hi,tol", [(32, False, -6.0, -2.0, 1e-4), (21, True, -6.0, -2.0, 1e-4),
                                                    (48, True, -3.5, -0.5, 2e-3)])
def test_train_kernels_fp32(gpu_device, T, with_state, lo, hi, tol):
    print(f"[case] train kernels fp32 T={T} state={with_state} w in [{lo},{hi}]", flush=True)
    B, H = 2, 3
    r, w, k, v, a, b = inputs(B, T, H, lo, hi, seed=T)
    g = torch.Generator().manual_seed(T + 1)
    dy = torch.randn(B, T, H, 64, generator=g)
    s0 = torch.randn(B, H, 64, 64, generator=g) * 0.1 if with_state else None
    ds_in = torch.randn(B, H, 64, 64, generator=g) * 0.1 if with_state else None

    y_o, sa_o, ck_o, S_o = otr.train_forward(r, w, k, v, a, b, s0=s0)
    grads_o = otr.train_backward(r, w, k, v, a, b, dy, ck_o, sa_o, ds_in=ds_in)

    d = lambda x: None if x is None else x.to(gpu_device).contiguous()
    rd, wd, kd, vd, ad, bd = (d(x) for x in (r, w, k, v, a, b))
    s_out = torch.empty(B, H, 64, 64, device=gpu_device) if with_state else None
    y, ck, sa = ops._train_forward(wd, rd, kd, vd, ad, bd, s0=d(s0), s_out=s_out)
    dw, dr, dk, dv, da, db, ds0 = ops._train_backward(wd, rd, kd, vd, ad, bd, d(dy), ck, sa, ds_in=d(ds_in),
                                                      want_ds0=with_state)
    torch.cuda.synchronize()
    assert close(y, y_o, tol) and close(sa, sa_o, tol) and close(ck, ck_o, tol)
    if with_state:
        assert close(s_out, S_o, tol)
    for name, got, ref in zip(("dr", "dw", "dk", "dv", "da", "db"), (dr, dw, dk, dv, da, db), grads_o[:6]):
        assert close(got, ref, tol), name
    if with_state:
        assert close(ds0, grads_o[6], tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_train_kernels_16bit_multichunk_strong_decay(gpu_device, dtype):
    """16-bit training op over T = 160 (five 32-token chunks of the chunked
    forward, ten 16-token segments of the backward) with raw decays in
    [-6, -0.5] (per-token decays down to 0.55, where the backward's step-back
    from the forward's checkpoints amplifies their error most), an initial state
    and a final-state gradient, against the float64 oracle on the rounded
    inputs.  y within one ulp + 2e-3 of max|y|; sa, checkpoints, final state and
    every gradient within 2e-2 of their largest magnitude."""
    print(f"[case] train kernels {dtype} T=160 strong decay", flush=True)
    B, T, H = 2, 160, 2
    xs = [x.to(dtype) for x in inputs(B, T, H, -6.0, -0.5, seed=77)]
    g = torch.Generator().manual_seed(78)
    dy = torch.randn(B, T, H, 64, generator=g).to(dtype)
    s0 = torch.randn(B, H, 64, 64, generator=g) * 0.1
    ds_in = torch.randn(B, H, 64, 64, generator=g) * 0.1
    r, w, k, v, a, b = (x.double() for x in xs)
    y_o, sa_o, ck_o, S_o = otr.train_forward(r, w, k, v, a, b, s0=s0.double())
    grads_o = otr.train_backward(r, w, k, v, a, b, dy.double(), ck_o, sa_o, ds_in=ds_in.double())

    d = lambda x: x.to(gpu_device).contiguous()
    rd, wd, kd, vd, ad, bd = (d(x) for x in xs)
    s_out = torch.empty(B, H, 64, 64, device=gpu_device)
    y, ck, sa = ops._train_forward(wd, rd, kd, vd, ad, bd, s0=d(s0), s_out=s_out)
    dw, dr, dk, dv, da, db, ds0 = ops._train_backward(wd, rd, kd, vd, ad, bd, d(dy), ck, sa, ds_in=d(ds_in),
                                                      want_ds0=True)
    torch.cuda.synchronize()
    assert y_close(y, y_o, dtype)
    assert close(sa, sa_o, 2e-2) and close(ck, ck_o, 2e-2) and close(s_out, S_o, 2e-2)
    for name, got, ref in zip(("dr", "dw", "dk", "dv", "da", "db"), (dr, dw, dk, dv, da, db), grads_o[:6]):
        assert close(got, ref, 2e-2), name
    assert close(ds0, grads_o[6], 2e-2)


def test_standard_training_operator_bf16(gpu_device):
    """load_wkv_operator('cuda', for_inference=False): RUN_CUDA_RWKV7g semantics
    (bf16 cast, [B, T, C] in and out, T % 16 asserted) and autograd gradients of
    every input against float64 autograd through the row-wise recurrence."""
    print("[case] standard training operator bf16", flush=True)
    op = ops.load_wkv_operator(device="cuda", for_inference=False, head_size=64)
    B, T, H = 2, 32, 2
    r, w, k, v, a, b = (x.bfloat16() for x in inputs(B, T, H, -6.0, -0.5, seed=5))
    g = torch.Generator().manual_seed(6)
    dy = torch.randn(B, T, H * 64, generator=g).bfloat16()
    flat = lambda x: x.reshape(B, T, H * 64)
    # reference: float64 autograd on the bf16-rounded inputs
    leaves = [flat(x).double().requires_grad_(True) for x in (r, w, k, v, a, b)]
    y_ref, _ = ow.wkv7_rowwise(*leaves)
    (y_ref * dy.double()).sum().backward()
    # operator: fp32 leaves on the GPU (the bf16 cast is part of the op's graph)
    dev_leaves = [flat(x).float().to(gpu_device).requires_grad_(True) for x in (r, w, k, v, a, b)]
    y = op(*dev_leaves)
    assert y.dtype == torch.bfloat16 and y.shape == (B, T, H * 64)
    (y.float() * dy.float().to(gpu_device)).sum().backward()
    torch.cuda.synchronize()
    ulp = torch.finfo(torch.bfloat16).eps
    dyv = (y.double().cpu() - y_ref.detach()).abs()
    assert bool((dyv <= ulp * y_ref.detach().abs() + 2e-3 * float(y_ref.detach().abs().max())).all())
    for name, got, ref in zip("rwkvab", dev_leaves, leaves):
        assert got.grad is not None and close(got.grad, ref.grad, 2e-2), name
    with pytest.raises(AssertionError):
        op(*(x[:, :20].detach() for x in dev_leaves))


def test_infctx_operator_chunks(gpu_device):
    """rwkv7_wkv_infctx: (y, final state) and gradients of the inputs and the
    initial state through two chained chunks equal one call over the whole
    sequence (the infinite-context use), and both match float64 autograd."""
    print("[case] infctx chunks", flush=True)
    B, T, H = 1, 40, 2
    xs = inputs(B, T, H, -6.0, -1.0, seed=9)
    g = torch.Generator().manual_seed(10)
    s0 = torch.randn(B, H, 64, 64, generator=g) * 0.1
    dy = torch.randn(B, T, H, 64, generator=g)
    dS = torch.randn(B, H, 64, 64, generator=g) * 0.1

    leaves = [x.double().requires_grad_(True) for x in xs]
    st = s0.double().requires_grad_(True)
    flat = lambda x: x.reshape(B, -1, H * 64)
    y_ref, S_ref = ow.wkv7_rowwise(*(flat(x) for x in leaves), state=st)
    ((flat(dy).double() * y_ref).sum() + (dS.double()[0] * S_ref[0]).sum()).backward()

    def run(split):
        r, w, k, v, a, b = (x.to(gpu_device).requires_grad_(True) for x in xs)
        state = s0.to(gpu_device).requires_grad_(True)
        ys, cur = [], state
        for lo, hi in ((0, split), (split, T)) if split else ((0, T),):
            y, cur = ops.rwkv7_wkv_infctx(w[:, lo:hi], r[:, lo:hi], k[:, lo:hi], v[:, lo:hi], a[:, lo:hi],
                                          b[:, lo:hi], state=cur)
            ys.append(y)
        y = torch.cat(ys, 1)
        ((y * dy.to(gpu_device)).sum() + (cur * dS.to(gpu_device)).sum()).backward()
        torch.cuda.synchronize()
        return y.detach(), cur.detach(), [x.grad for x in (r, w, k, v, a, b, state)]

    y1, S1, g1 = run(0)
    y2, S2, g2 = run(24)
    assert close(flat(y1), y_ref.detach(), 1e-4) and close(S1, S_ref.detach(), 1e-4)
    assert close(y2, y1, 1e-5) and close(S2, S1, 1e-5)
    for name, a1, a2, ref in zip(("r", "w", "k", "v", "a", "b", "s0"), g1, g2, [x.grad for x in leaves] + [st.grad]):
        assert close(a1, ref, 1e-4), name
        assert close(a2, a1, 1e-4), name


def test_infctx_raw_module(gpu_device):
    """load_hip_operator_infctx().forward / .backward (in place, as the
    reference's wkv7_infctx_op) agree with the autograd function."""
    B, T, H = 2, 19, 1
    xs = [x.to(gpu_device) for x in inputs(B, T, H, -6.0, -1.0, seed=12)]
    r, w, k, v, a, b = xs
    s0 = torch.randn(B, H, 64, 64, device=gpu_device) * 0.1
    dy = torch.randn(B, T, H, 64, device=gpu_device)
    mod = ops.load_hip_operator_infctx()
    s = s0.clone()
    y = torch.empty_like(r)
    mod.forward(w, r, k, v, a, b, s, y)
    grads = [torch.empty_like(x) for x in (w, r, k, v, a, b)] + [torch.empty_like(s0)]
    mod.backward(w, r, k, v, a, b, dy, s0, torch.empty(0, device=gpu_device), *grads)
    leaves = [x.clone().requires_grad_(True) for x in (w, r, k, v, a, b)]
    st = s0.clone().requires_grad_(True)
    y2, s2 = ops.rwkv7_wkv_infctx(*leaves, state=st)
    (y2 * dy).sum().backward()
    torch.cuda.synchronize()
    assert torch.equal(y, y2.detach()) and torch.equal(s, s2.detach())
    for got, ref in zip(grads, [x.grad for x in leaves] + [st.grad]):
        assert torch.equal(got, ref)


def test_train_kernels_fp16(gpu_device):
    """The fp16 instantiation of both kernels: inputs rounded to fp16 first, the
    oracle on the rounded values in float64; y and the gradients (fp16 outputs)
    within 2e-3 of their largest magnitude, sa and the checkpoints (float32) within
    1e-4.  T = 37 ends in a partial segment."""
    print("[case] train kernels fp16 T=37", flush=True)
    B, T, H = 2, 37, 2
    xs = [x.half() for x in inputs(B, T, H, -6.0, -1.0, seed=41)]
    g = torch.Generator().manual_seed(42)
    dy = torch.randn(B, T, H, 64, generator=g).half()
    r, w, k, v, a, b = (x.float() for x in xs)
    y_o, sa_o, ck_o, _ = otr.train_forward(r, w, k, v, a, b)
    grads_o = otr.train_backward(r, w, k, v, a, b, dy.float(), ck_o, sa_o)
    rd, wd, kd, vd, ad, bd = (x.to(gpu_device).contiguous() for x in xs)
    y, ck, sa = ops._train_forward(wd, rd, kd, vd, ad, bd)
    dw, dr, dk, dv, da, db, _ = ops._train_backward(wd, rd, kd, vd, ad, bd, dy.to(gpu_device), ck, sa)
    torch.cuda.synchronize()
    assert y.dtype == torch.float16
    assert close(y, y_o, 2e-3) and close(sa, sa_o, 1e-4) and close(ck, ck_o, 1e-4)
    for name, got, ref in zip(("dr", "dw", "dk", "dv", "da", "db"), (dr, dw, dk, dv, da, db), grads_o[:6]):
        assert got.dtype == torch.float16 and close(got, ref, 2e-3), name


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,with_state,strong", [(1, False, False), (10, True, False), (16, False, False),
                                                 (17, True, False), (32, False, False), (45, True, True),
                                                 (100, False, False), (64, True, True)])
def test_chunked_training_forward(gpu_device, dtype, T, with_state, strong):
    """16-bit inputs run the training forward in 32-token chunks on the matrix cores
    (one chunk = one set of contractions; the state after token 15 of a chunk and
    after its last token are the checkpoints).  Against the float64 oracle on the
    rounded inputs: y within one ulp of its type + 2e-3 of max|y|; sa, every
    checkpoint and the final state within 1e-4 of their largest magnitude.  T = 1,
    10, 17, 45, 100 end in partial chunks (and 10, 45 in partial 16-token segments);
    `strong` puts a log-decay below the kernel's matrix-form floor in one chunk,
    which that chunk then runs token by token."""
    print(f"[case] chunked training forward {dtype} T={T} state={with_state} strong={strong}", flush=True)
    B, H = 2, 3
    xs = inputs(B, T, H, -6.0, -0.5, seed=100 + T)
    if strong:
        xs[1][1, min(T - 1, 40), 2, 5] = 1.0  # decay exp(-e) per token, below the floor
    xs = [x.to(dtype) for x in xs]
    g = torch.Generator().manual_seed(200 + T)
    s0 = torch.randn(B, H, 64, 64, generator=g) * 0.1 if with_state else None
    r, w, k, v, a, b = (x.float() for x in xs)
    y_o, sa_o, ck_o, S_o = otr.train_forward(r, w, k, v, a, b, s0=s0)
    rd, wd, kd, vd, ad, bd = (x.to(gpu_device).contiguous() for x in xs)
    s_out = torch.empty(B, H, 64, 64, device=gpu_device) if with_state else None
    y, ck, sa = ops._train_forward(wd, rd, kd, vd, ad, bd, s0=None if s0 is None else s0.to(gpu_device),
                                   s_out=s_out)
    torch.cuda.synchronize()
    assert y.dtype == dtype and ck.shape == ck_o.shape
    assert y_close(y, y_o, dtype)
    assert close(sa, sa_o, 1e-4) and close(ck, ck_o, 1e-4)
    if with_state:
        assert close(s_out, S_o, 1e-4)


def test_training_forward_misaligned_inputs_token_serial(gpu_device):
    """Inputs not aligned to 4 elements take the token-serial forward: same
    results as the oracle (bf16, T = 21)."""
    print("[case] training forward misaligned bf16", flush=True)
    B, T, H = 1, 21, 2
    xs = [x.bfloat16() for x in inputs(B, T, H, -6.0, -1.0, seed=77)]
    r, w, k, v, a, b = (x.float() for x in xs)
    y_o, sa_o, ck_o, _ = otr.train_forward(r, w, k, v, a, b)

    def shifted(x):  # the same values one element past an aligned start
        buf = torch.empty(x.numel() + 1, dtype=x.dtype, device=gpu_device)
        buf[1:] = x.reshape(-1).to(gpu_device)
        return buf[1:].view(x.shape)

    rd, wd, kd, vd, ad, bd = (shifted(x) for x in xs)
    y, ck, sa = ops._train_forward(wd, rd, kd, vd, ad, bd)
    torch.cuda.synchronize()
    assert y_close(y, y_o, torch.bfloat16)
    assert close(sa, sa_o, 1e-4) and close(ck, ck_o, 1e-4)
