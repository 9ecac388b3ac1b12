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


MAX_VALID_ID = 65529  # last id of the reference vocabulary (rwkv_vocab_v20230424.txt)


def geometric_caps(n: int, mean: float, cap: int, g: torch.Generator):
    """``n`` stop lengths ~ Geometric(p = 1/mean) on {1, 2, ...}, clamped to ``cap``."""
    u = torch.rand(n, generator=g, dtype=torch.float64)
    caps = torch.clamp(torch.ceil(torch.log1p(-u) / torch.log1p(torch.tensor(-1.0 / mean))), 1, cap)
    return [int(c) for c in caps]


def cfg4_workload(seed: int = 4):
    """GRPO rollout inputs of the 1.5B benchmark: 64 prompts of U(256, 2048) ids in
    [1, 65529] and 64 x 8 per-path stop lengths ~ Geometric(mean 300) capped at 512."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(256, 2049, (64,), generator=g).tolist()
    prompts = [torch.randint(1, MAX_VALID_ID + 1, (L,), generator=g).tolist() for L in lens]
    return prompts, geometric_caps(64 * 8, 300.0, 512, g)


def cfg5_workload(seed: int = 5, n: int = 128, prompt_len: int = 2048):
    """7.2B rollout inputs: ``n`` prompts of ``prompt_len`` random ids and per-sequence
    stop lengths ~ Geometric(mean 600) capped at 1024."""
    g = torch.Generator().manual_seed(seed)
    prompts = [torch.randint(1, MAX_VALID_ID + 1, (prompt_len,), generator=g).tolist() for _ in range(n)]
    return prompts, geometric_caps(n, 600.0, 1024, g)
