"""Seeded synthetic inputs for the WKV7 op and the rollout.

All draws happen on the CPU with an explicit ``torch.Generator`` so the same seed
gives the same tensors on any machine; callers move them to the device.

Op inputs follow the benchmark definition of the isolated decode step and the
ragged prefill: r, k, v ~ N(0, 1); ``w`` is the op's *raw* decay input
``w_raw ~ U(-6, -1)`` (the op applies ``exp(-exp(w_raw))`` itself, as
``rwkvtune/models/rwkv7/operators/cuda/wkv7s.cu:27`` does, so the effective decay
lies in [0.692, 0.9975]); ``kk`` is N(0,1) L2-normalised per head; ``a = -kk`` and
``b = kk * iclr`` with ``iclr ~ U(0, 1)`` - the argument pattern of
``rwkvtune/models/rwkv7/model.py:246``.  The state is fp32 ~ N(0, 0.1^2).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class WkvInputs:
    r: torch.Tensor
    w: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    a: torch.Tensor
    b: torch.Tensor

    def as_tuple(self):
        return (self.r, self.w, self.k, self.v, self.a, self.b)

    def to(self, device=None, dtype=None):
        return WkvInputs(*(t.to(device=device, dtype=dtype) for t in self.as_tuple()))


def wkv_inputs(shape_prefix, H: int, N: int = 64, seed: int = 0,
               dtype=torch.bfloat16) -> WkvInputs:
    """Draw r, w, k, v, a, b of shape ``(*shape_prefix, H*N)`` in ``dtype``."""
    g = torch.Generator().manual_seed(seed)
    shp = tuple(shape_prefix) + (H * N,)
    r = torch.randn(shp, generator=g)
    k = torch.randn(shp, generator=g)
    v = torch.randn(shp, generator=g)
    w = torch.rand(shp, generator=g) * 5.0 - 6.0
    kk = torch.randn(tuple(shape_prefix) + (H, N), generator=g)
    kk = torch.nn.functional.normalize(kk, dim=-1, p=2.0).reshape(shp)
    iclr = torch.rand(shp, generator=g)
    a = -kk
    b = kk * iclr
    return WkvInputs(*(t.to(dtype) for t in (r, w, k, v, a, b)))


def wkv_state(n: int, H: int, N: int = 64, seed: int = 1, std: float = 0.1) -> torch.Tensor:
    """fp32 state ``[n, H, N, N]`` ~ N(0, std^2)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randn((n, H, N, N), generator=g) * std


def ragged_lengths(n: int, lo: int, hi: int, seed: int = 2):
    """``n`` integer lengths ~ U(lo, hi) inclusive, as a Python list."""
    g = torch.Generator().manual_seed(seed)
    return [int(x) for x in torch.randint(lo, hi + 1, (n,), generator=g)]


def cu_seqlens_of(lengths):
    cu = [0]
    for L in lengths:
        cu.append(cu[-1] + int(L))
    return cu
