"""Pins of the restated WKV7 training operator (oracle/wkv7_train.py) on the CPU:
forward against the row-wise WKV7 oracle, backward against torch autograd in
float64."""

import pytest
import torch

from oracle import wkv7 as ow
from oracle import wkv7_train as otr


def inputs(B, T, H, N=64, seed=0):
    g = torch.Generator().manual_seed(seed)
    shp = (B, T, H, N)
    r = torch.randn(shp, generator=g, dtype=torch.float64)
    k = torch.randn(shp, generator=g, dtype=torch.float64) * 0.5
    v = torch.randn(shp, generator=g, dtype=torch.float64)
    w = torch.rand(shp, generator=g, dtype=torch.float64) * -3.0 - 0.5      # decay in [0.61, 0.95]
    kk = torch.nn.functional.normalize(torch.randn(shp, generator=g, dtype=torch.float64), dim=-1)
    iclr = torch.rand(shp, generator=g, dtype=torch.float64)
    return r, w, k, v, -kk, kk * iclr


def flat(x):
    B, T, H, N = x.shape
    return x.reshape(B, T, H * N)


@pytest.mark.parametrize("T,seg", [(32, 16), (21, 16), (7, 1)])
def test_forward_matches_rowwise(T, seg):
    r, w, k, v, a, b = inputs(2, T, 2, seed=T)
    s0 = torch.randn(2, 2, 64, 64, dtype=torch.float64) * 0.1
    y, sa, ckpt, S = otr.train_forward(r, w, k, v, a, b, s0=s0, seg=seg)
    y_ref, S_ref = ow.wkv7_rowwise(*(flat(x) for x in (r, w, k, v, a, b)), state=s0)
    assert torch.allclose(flat(y), y_ref, atol=1e-12, rtol=1e-12)
    assert torch.allclose(S, S_ref, atol=1e-12, rtol=1e-12)
    assert torch.equal(ckpt[:, :, -1], S)                       # last checkpoint = final state
    if T >= 16 and seg == 16:
        y16, S16 = ow.wkv7_rowwise(*(flat(x[:, :16]) for x in (r, w, k, v, a, b)), state=s0)
        assert torch.allclose(ckpt[:, :, 0], S16, atol=1e-12)  # after token 15


@pytest.mark.parametrize("T,seg,with_state", [(32, 16, False), (21, 16, True), (9, 1, True)])
def test_backward_matches_autograd(T, seg, with_state):
    """Every gradient - inputs, initial state, and a loss on the final state -
    against autograd through the float64 row-wise recurrence."""
    r, w, k, v, a, b = inputs(1, T, 2, seed=100 + T)
    g = torch.Generator().manual_seed(7)
    dy = torch.randn(1, T, 2, 64, generator=g, dtype=torch.float64)
    s0 = torch.randn(1, 2, 64, 64, generator=g, dtype=torch.float64) * 0.1 if with_state else None
    ds_in = torch.randn(1, 2, 64, 64, generator=g, dtype=torch.float64) * 0.1 if with_state else None

    leaves = [x.clone().requires_grad_(True) for x in (r, w, k, v, a, b)]
    st = s0.clone().requires_grad_(True) if with_state else None
    y, S = ow.wkv7_rowwise(*(flat(x) for x in leaves), state=st)
    loss = (flat(dy) * y).sum()
    if with_state:
        loss = loss + (ds_in[0] * S).sum()
    loss.backward()

    _, sa, ckpt, _ = otr.train_forward(r, w, k, v, a, b, s0=s0, seg=seg)
    dr, dw, dk, dv, da, db, ds0 = otr.train_backward(r, w, k, v, a, b, dy, ckpt, sa, ds_in=ds_in, seg=seg)
    for got, leaf in zip((dr, dw, dk, dv, da, db), leaves):
        ref = leaf.grad
        assert torch.allclose(got, ref, atol=1e-9 * float(ref.abs().max()), rtol=1e-9)
    if with_state:
        assert torch.allclose(ds0, st.grad, atol=1e-9 * float(st.grad.abs().max()), rtol=1e-9)


def test_gradient_plants():
    """The autograd comparison catches a dropped term: the step-back and db
    without sa (zeroed saved sa) and the dS propagation without its a-term
    (zero a in the backward only) both move the gradients far from autograd."""
    r, w, k, v, a, b = inputs(1, 8, 1, seed=3)
    dy = torch.randn(1, 8, 1, 64, dtype=torch.float64, generator=torch.Generator().manual_seed(4))
    leaves = [x.clone().requires_grad_(True) for x in (r, w, k, v, a, b)]
    y, _ = ow.wkv7_rowwise(*(flat(x) for x in leaves))
    (flat(dy) * y).sum().backward()
    _, sa, ckpt, _ = otr.train_forward(r, w, k, v, a, b)
    no_sa = otr.train_backward(r, w, k, v, a, b, dy, ckpt, sa * 0)
    no_a = otr.train_backward(r, w, k, v, a * 0, b, dy, ckpt, sa)
    assert not torch.allclose(no_sa[5], leaves[5].grad, atol=1e-3)   # db
    assert not torch.allclose(no_a[1], leaves[1].grad, atol=1e-3)    # dw through the dS propagation
