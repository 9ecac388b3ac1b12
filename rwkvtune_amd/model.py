"""RWKV-7 model for the gfx950 rollout path.

Mirrors ``rwkvtune/models/rwkv7/model.py`` at the interface:

* the module tree and parameter names are the reference's (``emb``,
  ``blocks.{i}.ln0/ln1/ln2``, ``blocks.{i}.att.{x_r, ..., w0, w1, w2, a0, a1, a2,
  v0, v1, v2, g1, g2, k_k, k_a, r_k, receptance, key, value, output, ln_x}``,
  ``blocks.{i}.ffn.{x_k, key, value}``, ``ln_out``, ``head``; ``model.py:34-131,
  281-302, 346-365, 421-433``), so a reference ``state_dict`` loads unchanged;
* ``forward_with_state(idx, states)`` / ``init_state(B)`` / ``forward(idx,
  logits_to_keep)`` keep the reference's signatures and state layout
  (``model.py:435-520``).

The computation is not the reference's eager op chain.  A layer is five HIP
kernels from ``librwkv7_hip.so`` (residual + LayerNorm + token shift + lerps,
LoRA activations, the fused WKV time-mix, the FFN shift, relu^2) around the
dense projections, which are library GEMMs.  Every call works on a *slot pool*:
per layer ``att_kv [S, H, 64, 64]``, ``att_x_prev [S, C]``, ``ffn_x_prev [S, C]``,
all float32, addressed by slot index, so the engine never gathers or scatters
states (``rwkvtune/inference/scheduler_core.py:377-395``).

Element-wise math is float32 for every model dtype; the dense projections run
in the model dtype with float32 accumulation.  There is no CPU path: the HIP
library must be present (``_lib.HipLibraryMissing`` otherwise).
"""

from __future__ import annotations

import ctypes
import math
import weakref
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from . import operators as wkv_ops

HEAD_SIZE = 64


@dataclass
class RWKV7Config:
    """Model fields of the reference's ``SimpleTrainConfig``
    (``rwkvtune/models/rwkv7/config.py:7-79``, exported as ``RWKV7Config``)."""
    n_layer: int = 12
    n_embd: int = 768
    vocab_size: int = 65536
    ctx_len: int = 1024
    head_size_a: int = 64
    dim_att_lora: int = 0
    dim_gate_lora: int = 0
    dim_mv_lora: int = 0
    dim_att: int = field(init=False)

    def __post_init__(self):
        self.dim_att = self.n_embd
        if self.head_size_a != HEAD_SIZE:
            raise ValueError(f"head_size_a must be {HEAD_SIZE}")
        if self.n_embd % (4 * HEAD_SIZE) != 0:
            raise ValueError("n_embd must be a multiple of 256 (H a multiple of 4)")

    @property
    def n_head(self) -> int:
        return self.n_embd // HEAD_SIZE

    def lora_dims(self):
        """(decay, a, value, gate) LoRA ranks; the defaults are the reference's
        formulas (``model.py:71-99``)."""
        C = self.n_embd
        dw = self.dim_att_lora if self.dim_att_lora > 0 else max(32, int(round((2.0 * C ** 0.5) / 32) * 32))
        dv = self.dim_mv_lora if self.dim_mv_lora > 0 else max(32, int(round((1.4 * C ** 0.5) / 32) * 32))
        dg = self.dim_gate_lora if self.dim_gate_lora > 0 else max(32, int(round((5.6 * C ** 0.5) / 32) * 32))
        return dw, dw, dv, dg


# Model presets of the benchmark configurations (architecture and LoRA ranks of
# rwkvtune/configs/models/rwkv7-{0.1b,1.5b,7.2b}.json).  cfg1 keeps the
# reference's default LoRA formula (dim_* = 0).
PRESETS = {
    "rwkv7-0.1b": dict(n_layer=12, n_embd=768),
    "rwkv7-0.4b": dict(n_layer=24, n_embd=1024, dim_att_lora=64, dim_gate_lora=128, dim_mv_lora=32),
    "rwkv7-1.5b": dict(n_layer=24, n_embd=2048, dim_att_lora=96, dim_gate_lora=256, dim_mv_lora=64),
    "rwkv7-2.9b": dict(n_layer=32, n_embd=2560, dim_att_lora=96, dim_gate_lora=320, dim_mv_lora=64),
    "rwkv7-7.2b": dict(n_layer=32, n_embd=4096, dim_att_lora=128, dim_gate_lora=480, dim_mv_lora=96),
}


def config_from_preset(name: str, **over) -> RWKV7Config:
    kw = dict(PRESETS[name])
    kw.update(over)
    return RWKV7Config(**kw)


class RWKV7TimeMix(nn.Module):
    """Parameter container of ``RWKV7TimeMix`` (``model.py:34-131``)."""

    def __init__(self, config: RWKV7Config, layer_id: int):
        super().__init__()
        C, H, N = config.n_embd, config.n_head, HEAD_SIZE
        dw, da, dv, dg = config.lora_dims()
        self.layer_id = layer_id
        self.head_size = N
        self.n_head = H
        for name in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g", "w0", "a0", "k_k", "k_a"):
            setattr(self, name, nn.Parameter(torch.empty(1, 1, C)))
        self.w1 = nn.Parameter(torch.empty(C, dw))
        self.w2 = nn.Parameter(torch.empty(dw, C))
        self.a1 = nn.Parameter(torch.empty(C, da))
        self.a2 = nn.Parameter(torch.empty(da, C))
        if layer_id > 0:
            self.v0 = nn.Parameter(torch.empty(1, 1, C))
            self.v1 = nn.Parameter(torch.empty(C, dv))
            self.v2 = nn.Parameter(torch.empty(dv, C))
        self.g1 = nn.Parameter(torch.empty(C, dg))
        self.g2 = nn.Parameter(torch.empty(dg, C))
        self.r_k = nn.Parameter(torch.empty(H, N))
        self.receptance = nn.Linear(C, C, bias=False)
        self.key = nn.Linear(C, C, bias=False)
        self.value = nn.Linear(C, C, bias=False)
        self.output = nn.Linear(C, C, bias=False)
        self.ln_x = nn.GroupNorm(H, C, eps=64e-5)


class RWKV7ChannelMix(nn.Module):
    """Parameter container of ``RWKV7ChannelMix`` (``model.py:281-302``)."""

    def __init__(self, config: RWKV7Config, layer_id: int):
        super().__init__()
        C = config.n_embd
        self.layer_id = layer_id
        self.x_k = nn.Parameter(torch.empty(1, 1, C))
        self.key = nn.Linear(C, 4 * C, bias=False)
        self.value = nn.Linear(4 * C, C, bias=False)


class RWKV7Block(nn.Module):
    """Parameter container of ``RWKV7Block`` (``model.py:346-365``)."""

    def __init__(self, config: RWKV7Config, layer_id: int):
        super().__init__()
        self.layer_id = layer_id
        self.ln1 = nn.LayerNorm(config.n_embd)
        self.ln2 = nn.LayerNorm(config.n_embd)
        self.skip_ln0 = False
        if layer_id == 0:
            self.ln0 = nn.LayerNorm(config.n_embd)
        self.att = RWKV7TimeMix(config, layer_id)
        self.ffn = RWKV7ChannelMix(config, layer_id)


# ---------------------------------------------------------------------------
# Seeded dense initialisation
# ---------------------------------------------------------------------------

@torch.no_grad()
def init_dense_(model: "RWKV7Model", seed: int = 0, device=None) -> "RWKV7Model":
    """Seeded dense random init.

    The per-channel structured parameters follow the reference formulas
    (``model.py:48-104, 288-293``); every matrix (and the embedding) is drawn
    N(0, (0.5/sqrt(fan_in))^2) instead of the reference's zero / orthogonal init
    (the reference zeroes ``output``, ``ffn.value`` and the LoRA down
    projections, ``model.py:76-117, 302``, which would make every logit
    independent of the recurrence).  LayerNorm / GroupNorm weights are
    1 + N(0, 0.1^2) and biases N(0, 0.1^2), so every parameter reaches the output.
    Draws happen on ``device`` (default: the model's) with a seeded generator.
    """
    cfg = model.config
    dev = torch.device(device) if device is not None else next(model.parameters()).device
    gen = torch.Generator(device=dev).manual_seed(seed)
    C, N, L = cfg.n_embd, HEAD_SIZE, cfg.n_layer

    def normal_(p, std):
        p.copy_(torch.randn(p.shape, generator=gen, device=dev, dtype=torch.float32) * std)

    def mat_(p, fan_in):
        normal_(p, 0.5 / math.sqrt(fan_in))

    ddd = torch.arange(C, dtype=torch.float64, device=dev) / C
    n = torch.arange(C, dtype=torch.float64, device=dev)
    linear = n / (C - 1) - 0.5
    zig = ((n % N) - (N - 1) / 2) / ((N - 1) / 2)
    zig = zig * zig.abs()

    def set_(p, v):
        p.copy_(v.reshape(p.shape).to(torch.float32))

    normal_(model.emb.weight, 1.0)
    for i, blk in enumerate(model.blocks):
        r01 = i / (L - 1) if L > 1 else 0.0
        r1a0 = 1.0 - i / L
        att, ffn = blk.att, blk.ffn
        for ln in [blk.ln1, blk.ln2] + ([blk.ln0] if i == 0 else []):
            set_(ln.weight, 1.0 + 0.1 * torch.randn(C, generator=gen, device=dev))
            set_(ln.bias, 0.1 * torch.randn(C, generator=gen, device=dev))
        set_(att.x_r, 1.0 - ddd ** (0.2 * r1a0))
        set_(att.x_w, 1.0 - ddd ** (0.9 * r1a0))
        set_(att.x_k, 1.0 - ddd ** (0.7 * r1a0))
        set_(att.x_v, 1.0 - ddd ** (0.7 * r1a0))
        set_(att.x_a, 1.0 - ddd ** (0.9 * r1a0))
        set_(att.x_g, 1.0 - ddd ** (0.2 * r1a0))
        www = -6 + 6 * (n / (C - 1)) ** (1 + 1 * r01 ** 0.3)
        set_(att.w0, www + 0.5 + zig * 2.5)
        set_(att.a0, -0.19 + zig * 0.3 + linear * 0.4)
        if i > 0:
            set_(att.v0, 0.73 - linear * 0.4)
        set_(att.k_k, 0.71 - linear * 0.1)
        set_(att.k_a, torch.full((C,), 1.02, dtype=torch.float64, device=dev))
        set_(att.r_k, torch.full((C,), -0.04, dtype=torch.float64, device=dev))
        for name in ("w1", "a1", "g1") + (("v1",) if i > 0 else ()):
            mat_(getattr(att, name), C)
        for name in ("w2", "a2", "g2") + (("v2",) if i > 0 else ()):
            p = getattr(att, name)
            mat_(p, p.shape[0])
        for lin in (att.receptance, att.key, att.value, att.output, ffn.key, ffn.value):
            mat_(lin.weight, lin.weight.shape[1])
        set_(att.ln_x.weight, 1.0 + 0.1 * torch.randn(C, generator=gen, device=dev))
        set_(att.ln_x.bias, 0.1 * torch.randn(C, generator=gen, device=dev))
        set_(ffn.x_k, 1.0 - ddd ** (r1a0 ** 4))
    set_(model.ln_out.weight, 1.0 + 0.1 * torch.randn(C, generator=gen, device=dev))
    set_(model.ln_out.bias, 0.1 * torch.randn(C, generator=gen, device=dev))
    mat_(model.head.weight, C)
    model.invalidate()
    return model


# ---------------------------------------------------------------------------
# Slot pool
# ---------------------------------------------------------------------------

class StatePool:
    """Per-layer recurrent state of ``n_slots`` sequences, float32:
    ``kv [L, S, H, 64, 64]``, ``att_x [L, S, C]``, ``ffn_x [L, S, C]``
    (the pool of ``scheduler_core.py:180-205``, with x_prev kept in float32)."""

    def __init__(self, config: RWKV7Config, n_slots: int, device):
        L, C, H = config.n_layer, config.n_embd, config.n_head
        self.n_slots = n_slots
        self.kv = torch.zeros((L, n_slots, H, HEAD_SIZE, HEAD_SIZE), dtype=torch.float32, device=device)
        self.att_x = torch.zeros((L, n_slots, C), dtype=torch.float32, device=device)
        self.ffn_x = torch.zeros((L, n_slots, C), dtype=torch.float32, device=device)

    def zero_(self, slots=None):
        if slots is None:
            self.kv.zero_()
            self.att_x.zero_()
            self.ffn_x.zero_()
        else:
            self.kv[:, slots] = 0
            self.att_x[:, slots] = 0
            self.ffn_x[:, slots] = 0

    def copy_slots_(self, dst_slots, src: "StatePool", src_slots):
        """dst[dst_slots] <- src[src_slots] on every layer (index tensors on device)."""
        self.kv[:, dst_slots] = src.kv[:, src_slots]
        self.att_x[:, dst_slots] = src.att_x[:, src_slots]
        self.ffn_x[:, dst_slots] = src.ffn_x[:, src_slots]


# ---------------------------------------------------------------------------
# The model
# ---------------------------------------------------------------------------

class PackedWeight:
    """An nn.Linear weight [N][K] (bf16) in the tiled layout of the decode GEMM
    (``rwkv7_gemm_pack``): 64 x 64 tiles, each one contiguous 8 KB block, so a
    K step of the GEMM reads one linear piece of HBM instead of 64 row segments."""

    def __init__(self, weight: torch.Tensor):
        if weight.dtype != torch.bfloat16 or weight.ndim != 2 or weight.stride(1) != 1:
            raise ValueError("PackedWeight needs a bf16 [N][K] weight with unit column stride")
        self.N, self.K = int(weight.shape[0]), int(weight.shape[1])
        n = _lib.load().rwkv7_gemm_packed_elems(self.N, self.K)
        if n < 0:
            raise ValueError("rwkv7_gemm_packed_elems: " + _lib.load().rwkv7_last_error().decode())
        self.t = torch.empty(n, dtype=torch.bfloat16, device=weight.device)
        self.pack(weight)

    def pack(self, weight: torch.Tensor):
        """(Re)write the packed copy from ``weight`` (same shape) into the same buffer."""
        if tuple(weight.shape) != (self.N, self.K):
            raise ValueError(f"repack of a {self.N} x {self.K} weight from {tuple(weight.shape)}")
        w = weight if weight.stride(0) % 8 == 0 and weight.data_ptr() % 16 == 0 else weight.contiguous()
        _lib.call("rwkv7_gemm_pack", _lib.ptr(w), w.stride(0), self.N, self.K, _lib.ptr(self.t),
                  _lib.stream_of(self.t))


class HeadPack:
    """The head weight [V][K] (bf16) in the layout of ``rwkv7_head_pack``
    (64-row x 32-column pieces of 4 KB), for ``rwkv7_head_logits``: the logits
    of up to ``MAX_ROWS`` rows (decode steps, prefill's last tokens) in one
    launch that streams the weight once.  Above that a library GEMM with
    256-row tiles is faster (LM head 65,536 x 2,048, cold weights: 48-55 us
    against 67-72 us for the library at 32-128 rows; 75 us for both at 192
    rows; the library ahead at 256)."""

    MAX_ROWS = 128

    @staticmethod
    def supported(weight: torch.Tensor) -> bool:
        V, K = weight.shape
        return (weight.dtype == torch.bfloat16 and weight.ndim == 2 and weight.is_cuda and V % 256 == 0
                and K % 64 == 0 and 256 <= K <= 65536)

    def __init__(self, weight: torch.Tensor):
        if not self.supported(weight):
            raise ValueError("HeadPack needs a bf16 [V][K] weight on the GPU with V % 256 == 0, K % 64 == 0, "
                             "256 <= K <= 65536")
        self.V, self.K = int(weight.shape[0]), int(weight.shape[1])
        n = _lib.load().rwkv7_head_packed_elems(self.V, self.K)
        if n < 0:
            raise ValueError("rwkv7_head_packed_elems: " + _lib.load().rwkv7_last_error().decode())
        self.t = torch.empty(n, dtype=torch.bfloat16, device=weight.device)
        self.pack(weight)

    def pack(self, weight: torch.Tensor):
        """(Re)write the packed copy from ``weight`` (same shape) into the same buffer."""
        if tuple(weight.shape) != (self.V, self.K):
            raise ValueError(f"repack of a {self.V} x {self.K} head from {tuple(weight.shape)}")
        w = weight if weight.stride(1) == 1 and weight.stride(0) % 8 == 0 and weight.data_ptr() % 16 == 0 \
            else weight.contiguous()
        _lib.call("rwkv7_head_pack", _lib.ptr(w), w.stride(0), self.V, self.K, _lib.ptr(self.t),
                  _lib.stream_of(self.t))

    def logits(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x [M, K] bf16 (unit column stride) -> logits [M, V] bf16 (into ``out``
        if given: [M, >= V] bf16 with unit column stride)."""
        M = x.shape[0]
        if out is None:
            out = torch.empty((M, self.V), dtype=torch.bfloat16, device=x.device)
        _lib.call("rwkv7_head_logits", M, self.V, self.K, _lib.ptr(x), x.stride(0), _lib.ptr(self.t),
                  _lib.ptr(out), out.stride(0), _lib.stream_of(x))
        return out


class _LayerPack:
    """float32 copies of one layer's per-channel parameters, laid out for the
    kernels, and (bf16 models) the packed decode-GEMM weights.  ``refresh``
    rewrites every copy from the current parameters into the same buffers, so
    kernel argument pointers (and the pointer table ``tparams``) stay valid."""

    def __init__(self, blk: RWKV7Block, C: int):
        self.C = C
        self.layer0 = blk.layer_id == 0
        self.gp = {}
        self._fill(blk, alloc=True)

    def refresh(self, blk: RWKV7Block):
        self._fill(blk, alloc=False)

    @staticmethod
    def _f32(t):
        return t.detach().reshape(-1).to(torch.float32).contiguous()

    def _set(self, name, value, alloc):
        if alloc:
            setattr(self, name, value)
        else:
            getattr(self, name).copy_(value)

    def _fill(self, blk: RWKV7Block, alloc: bool):
        att, ffn = blk.att, blk.ffn
        C = self.C
        f32 = self._f32
        use_ln0 = self.layer0 and not blk.skip_ln0
        if alloc:
            self.use_ln0 = use_ln0
        elif use_ln0 != self.use_ln0:
            raise RuntimeError("skip_ln0 changed: rebuild the packs")
        if use_ln0:
            self._set("ln0_w", f32(blk.ln0.weight), alloc)
            self._set("ln0_b", f32(blk.ln0.bias), alloc)
        self.ln0 = (self.ln0_w, self.ln0_b) if use_ln0 else None
        for nm, ln in (("ln1", blk.ln1), ("ln2", blk.ln2)):
            self._set(nm + "_w", f32(ln.weight), alloc)
            self._set(nm + "_b", f32(ln.bias), alloc)
        self.ln1 = (self.ln1_w, self.ln1_b)
        self.ln2 = (self.ln2_w, self.ln2_b)
        # seven mixes, in the order the projections consume them: r, k, v (one
        # batched GEMM), then the LoRA inputs w, a, g, v (one batched GEMM)
        self._set("mix7", torch.stack([f32(getattr(att, n)) for n in ("x_r", "x_k", "x_v", "x_w", "x_a", "x_g",
                                                                        "x_v")]), alloc)
        self._set("mixk", f32(ffn.x_k).reshape(1, C), alloc)
        dev = self.mix7.device
        zero = torch.zeros(C, dtype=torch.float32, device=dev)
        tv = [f32(att.w0), f32(att.a0), f32(att.v0) if not self.layer0 else zero,
              f32(att.k_k), f32(att.k_a), f32(att.r_k), f32(att.ln_x.weight), f32(att.ln_x.bias)]
        if alloc:
            self.tvecs = tv
            ptrs = [t.data_ptr() for t in self.tvecs]
            if self.layer0:
                ptrs[2] = 0
            self.tparams = (ctypes.c_void_p * 8)(*ptrs)
        else:
            for dst, src in zip(self.tvecs, tv):
                dst.copy_(src)
        # Batched projection weights ([batch][in][out], contiguous: the right
        # operand of a batched GEMM must not be a transposed view): r/k/v, and the
        # LoRA pairs zero-padded to a common rank D (padded down-columns give 0,
        # whose activation meets zero up-rows, so padding adds nothing).
        with torch.no_grad():
            downs = [att.w1, att.a1, att.g1] + ([] if self.layer0 else [att.v1])
            ups = [att.w2, att.a2, att.g2] + ([] if self.layer0 else [att.v2])
            if alloc:
                D = max(d.shape[1] for d in downs)
                D = (D + 31) // 32 * 32
                dt = att.w1.dtype
                self.lora_down = torch.zeros((len(downs), C, D), dtype=dt, device=att.w1.device)
                self.lora_up = torch.zeros((len(ups), D, C), dtype=dt, device=att.w1.device)
            for i, (dn, up) in enumerate(zip(downs, ups)):
                self.lora_down[i, :, :dn.shape[1]] = dn.detach()
                self.lora_up[i, :up.shape[0], :] = up.detach()
        # decode-GEMM weights of bf16 models, packed: r / k / v, the LoRA downs
        # and ups as [out][in] matrices, the output projection, the FFN key and value
        if att.w1.dtype == torch.bfloat16:
            with torch.no_grad():
                mats = {"r": att.receptance.weight, "k": att.key.weight, "v": att.value.weight,
                        "o": att.output.weight, "fk": ffn.key.weight, "fv": ffn.value.weight}
                names = ("w1", "a1", "g1", "w2", "a2", "g2") + (() if self.layer0 else ("v1", "v2"))
                for n in names:
                    mats[n] = getattr(att, n).detach().t().contiguous()
                for n, wt in mats.items():
                    if alloc:
                        self.gp[n] = PackedWeight(wt.detach())
                    else:
                        self.gp[n].pack(wt.detach())


class RWKV7Model(nn.Module):
    """RWKV-7 language model on the HIP library (interface of ``model.py:421-520``)."""

    def __init__(self, config: RWKV7Config):
        super().__init__()
        self.config = config
        self.emb = nn.Embedding(config.vocab_size, config.n_embd)
        self.blocks = nn.ModuleList([RWKV7Block(config, i) for i in range(config.n_layer)])
        self.ln_out = nn.LayerNorm(config.n_embd)
        self.head = nn.Linear(config.n_embd, config.vocab_size, bias=False)
        self._packs = None
        self._head_pack = None
        self._packs_key = None
        self._packs_struct = None
        # bumped whenever the packs are rebuilt (new buffers) or a parameter's
        # storage moved: captured decode graphs hold both kinds of address
        self._packs_gen = 0
        # called before the parameter check of every packs(): refreshes the
        # merged weights of a caller's LoRA-wrapped linears (as_hip_model)
        self._pre_pack = None
        # decode rows of a bf16 model run their projections on the library's
        # grouped MFMA GEMM over packed weights: r, k, v and the LoRA downs (tanh /
        # sigmoid fused) in one launch, the LoRA ups in one, the FFN key (relu^2
        # fused) and value, the output projection (split-K planes summed by the
        # next row kernel)
        self.use_grouped_gemm = True
        # logits of up to HeadPack.MAX_ROWS rows of a bf16 model on the library's
        # head GEMM over a packed copy of the head weight (larger row counts and
        # other dtypes: a library GEMM)
        self.use_head_kernel = True
        # decode: output projection on the grouped GEMM's split-K planes (summed by
        # the next row kernel) instead of the library GEMM
        self.use_grouped_output = True
        self._lora_h = {}

    # -- bookkeeping ---------------------------------------------------------

    def invalidate(self):
        """Drop the cached parameter packs; the next forward rebuilds them.  (Not
        needed after in-place parameter updates, which ``packs`` detects.)"""
        self._packs = None

    def _apply(self, fn, *args, **kwargs):
        self._packs = None
        return super()._apply(fn, *args, **kwargs)

    def load_state_dict(self, state_dict, strict: bool = True, assign: bool = False):
        """Loads a reference state dict: ``r_k`` may be flat (``model.py:577-584``);
        layer-0 ``v0/v1/v2`` are dropped (``model.py:586-599``); without ``ln0`` in
        the source the embedding is taken as already normalised (``skip_ln0``,
        ``model.py:601-609``)."""
        sd = dict(state_dict)
        H, N = self.config.n_head, HEAD_SIZE
        for key in list(sd):
            if key.endswith("att.r_k") and sd[key].ndim == 1:
                sd[key] = sd[key].view(H, N)
        for s in ("0", "1", "2"):
            sd.pop(f"blocks.0.att.v{s}", None)
        has_ln0 = "blocks.0.ln0.weight" in state_dict and "blocks.0.ln0.bias" in state_dict
        res = super().load_state_dict(sd, strict=False, assign=assign)
        if len(self.blocks) > 0:
            self.blocks[0].skip_ln0 = not has_ln0
        self.invalidate()
        return res

    @property
    def device(self):
        return self.emb.weight.device

    @property
    def dtype(self):
        return self.emb.weight.dtype

    def _check_device(self):
        if self.device.type != "cuda":
            raise RuntimeError("RWKV7Model runs on the HIP library only; move it to a GPU device first")
        _lib.load()

    def _param_key(self):
        """(data_ptr, version) of every parameter: an in-place update (an
        optimizer step, ``copy_``, ``mul_`` ...) bumps the version, a move or
        reassignment changes the pointer."""
        return tuple((p.data_ptr(), p._version) for p in self.parameters())

    def _struct_key(self):
        return (tuple((p.device, p.dtype, tuple(p.shape)) for p in self.parameters()),
                tuple(b.skip_ln0 for b in self.blocks))

    def packs(self):
        """The kernels' parameter packs, rebuilt or refreshed whenever a parameter
        changed since they were made (no ``invalidate()`` needed after an
        optimizer step that updates the parameters in place)."""
        if self._pre_pack is not None:
            self._pre_pack()
        key = self._param_key()
        if self._packs is not None and key == self._packs_key:
            return self._packs
        self._check_device()
        old = self._packs_key
        C = self.config.n_embd
        with torch.no_grad():
            if self._packs is not None and self._struct_key() == self._packs_struct:
                for pk, b in zip(self._packs, self.blocks):
                    pk.refresh(b)
                self._ln_out[0].copy_(self.ln_out.weight.detach().float())
                self._ln_out[1].copy_(self.ln_out.bias.detach().float())
                if self._head_pack is not None:
                    self._head_pack.pack(self.head.weight.detach())
            else:
                self._packs = [_LayerPack(b, C) for b in self.blocks]
                self._ln_out = (self.ln_out.weight.detach().float().contiguous(),
                                self.ln_out.bias.detach().float().contiguous())
                self._head_pack = None
                if HeadPack.supported(self.head.weight):
                    self._head_pack = HeadPack(self.head.weight.detach())
                self._packs_struct = self._struct_key()
                self._packs_gen += 1
        if old is not None and [k[0] for k in key] != [k[0] for k in old]:
            # the embedding and the head are read in place by the decode step
            self._packs_gen += 1
        self._packs_key = key
        return self._packs

    def init_state(self, batch_size: int):
        """Per-layer states as in ``model.py:499-520`` (x_prev in float32 here)."""
        C, H, N = self.config.n_embd, self.config.n_head, HEAD_SIZE
        dev = self.device
        return [{"att_x_prev": torch.zeros(batch_size, C, dtype=torch.float32, device=dev),
                 "att_kv": torch.zeros(batch_size, H, N, N, dtype=torch.float32, device=dev),
                 "ffn_x_prev": torch.zeros(batch_size, C, dtype=torch.float32, device=dev)}
                for _ in range(self.config.n_layer)]

    # -- pooled forward ------------------------------------------------------

    def _lin(self, x, weight):
        return F.linear(x, weight)

    class GemmWorkspace:
        """Split-K partial tiles of the grouped decode GEMM (float32).  Launches
        that share it must be ordered (one stream)."""

        def __init__(self, device, floats: int = 1 << 22):
            self.ws = torch.empty(floats, dtype=torch.float32, device=device)

        def ensure(self, floats: int):
            if floats > self.ws.numel():
                self.ws = torch.empty(max(floats, 2 * self.ws.numel()), dtype=torch.float32, device=self.ws.device)

    _gemm_ws = {}

    @staticmethod
    def gemm_workspace(dev) -> "RWKV7Model.GemmWorkspace":
        """The device's shared split-K workspace (created on first use)."""
        ws = RWKV7Model._gemm_ws.get(dev)
        if ws is None:
            ws = RWKV7Model._gemm_ws[dev] = RWKV7Model.GemmWorkspace(dev)
        return ws

    @staticmethod
    def _gemm_group(M: int, probs, stream):
        """One grouped decode-GEMM launch: probs = [(A, B, C, epi)] with B a
        ``PackedWeight``; C = epi(A . B^T), A [M][B.K] and C [M][B.N] bf16 views
        with unit column stride."""
        n = len(probs)
        P = ctypes.c_void_p
        dev = probs[0][0].device
        for a, b, c, _ in probs:
            if (a.dtype != torch.bfloat16 or c.dtype != torch.bfloat16 or a.shape != (M, b.K)
                    or c.shape != (M, b.N) or a.stride(1) != 1 or c.stride(1) != 1):
                raise ValueError(f"grouped GEMM operands: A {tuple(a.shape)} {a.dtype}, C {tuple(c.shape)} "
                                 f"{c.dtype} for a {b.N} x {b.K} weight and M = {M}")
        arrA = (P * n)(*[a.data_ptr() for a, _, _, _ in probs])
        arrB = (P * n)(*[b.t.data_ptr() for _, b, _, _ in probs])
        arrC = (P * n)(*[c.data_ptr() for _, _, c, _ in probs])
        lda = (ctypes.c_int64 * n)(*[a.stride(0) for a, _, _, _ in probs])
        ldc = (ctypes.c_int64 * n)(*[c.stride(0) for _, _, c, _ in probs])
        N = (ctypes.c_int * n)(*[b.N for _, b, _, _ in probs])
        K = (ctypes.c_int * n)(*[b.K for _, b, _, _ in probs])
        epi = (ctypes.c_int * n)(*[x for _, _, _, x in probs])
        need = _lib.load().rwkv7_gemm_decode_workspace(M, n, N, K)
        if need < 0:
            raise ValueError("rwkv7_gemm_decode_workspace: " + _lib.load().rwkv7_last_error().decode())
        ws = RWKV7Model._gemm_ws.get(dev)
        if ws is None:
            ws = RWKV7Model._gemm_ws[dev] = RWKV7Model.GemmWorkspace(dev)
        ws.ensure(need)
        _lib.call("rwkv7_gemm_decode", M, n, arrA, arrB, arrC, lda, ldc, N, K, epi,
                  P(ws.ws.data_ptr()), ws.ws.numel(), stream)

    @staticmethod
    def _gemm_partials(M: int, a, b, stream):
        """The grouped GEMM's K-range partial products of A . B^T (B a
        ``PackedWeight``) left as float32 planes [P][M][B.N] in the shared
        workspace; returns (workspace tensor, P).  The next row kernel sums
        them (``add_parts``) in place of the reduction launch."""
        if a.dtype != torch.bfloat16 or a.shape != (M, b.K) or a.stride(1) != 1:
            raise ValueError(f"grouped GEMM operand: A {tuple(a.shape)} {a.dtype} for a {b.N} x {b.K} weight")
        lib = _lib.load()
        parts = lib.rwkv7_gemm_decode_partial_count(M, b.N, b.K)
        if parts < 1:
            raise ValueError("rwkv7_gemm_decode_partial_count: " + lib.rwkv7_last_error().decode())
        dev = a.device
        ws = RWKV7Model._gemm_ws.get(dev)
        if ws is None:
            ws = RWKV7Model._gemm_ws[dev] = RWKV7Model.GemmWorkspace(dev)
        ws.ensure(parts * M * b.N)
        got = ctypes.c_int32(0)
        _lib.call("rwkv7_gemm_decode_partials", M, _lib.ptr(a), _lib.ptr(b.t), a.stride(0), b.N, b.K,
                  _lib.ptr(ws.ws), ws.ws.numel(), ctypes.c_void_p(ctypes.addressof(got)), stream)
        return ws.ws, got.value

    @torch.no_grad()
    def forward_pooled(self, tokens: torch.Tensor, row_slot: torch.Tensor, row_last: torch.Tensor,
                       pool: StatePool, *, decode: bool, cu_seqlens: Optional[torch.Tensor] = None,
                       seq_slot: Optional[torch.Tensor] = None,
                       logit_rows: Optional[torch.Tensor] = None, n_logit_rows: Optional[int] = None,
                       return_hidden: bool = False):
        """Run every layer over ``M`` packed rows on the slot pool.

        tokens [M] int64; row_slot / row_last [M] int32 (see ``rwkv7_shift_mix``).
        decode=True: one token per sequence (row m is sequence m), fused WKV
        time-mix.  decode=False: ragged prefill; ``cu_seqlens`` [nseq+1] and
        ``seq_slot`` [nseq] int32 describe the sequences.  ``logit_rows``: int32
        rows whose logits are returned (None: all rows).  No host synchronisation.
        """
        cfg = self.config
        C, H, L = cfg.n_embd, cfg.n_head, cfg.n_layer
        M = tokens.shape[0]
        dt = self.dtype
        code = _lib.dtype_code(dt)
        dev = tokens.device
        st = _lib.stream_of(tokens)
        P = _lib.ptr
        packs = self.packs()
        if M == 0:
            raise ValueError("forward_pooled needs at least one row")

        x_res = torch.empty((M, C), dtype=torch.float32, device=dev)
        x_mid = torch.empty((M, C), dtype=torch.float32, device=dev)
        mixes = torch.empty((7, M, C), dtype=dt, device=dev)
        xk_ffn = torch.empty((1, M, C), dtype=dt, device=dev)
        v_first = torch.empty((M, C), dtype=torch.float32, device=dev)
        if not decode:
            # prefill WKV operands and output in the model dtype, as the reference
            # passes them to its WKV kernel (model.py:233-250); bf16 / fp16 models
            # then take the 16-bit chunked matrix-core kernel
            # w, k', v', -kk, kk*a; r goes to the WKV op as the projection wrote it
            ops = torch.empty((5, M, C), dtype=dt, device=dev)
            ops_ptrs = (ctypes.c_void_p * 6)(None, *[ops[i].data_ptr() for i in range(5)])
            y = torch.empty((M, C), dtype=dt, device=dev)
        ffn_out = None
        ffn_parts, ffn_stride = 0, 0  # > 0: ffn_out holds the FFN value's float32 partial planes
        S = pool.n_slots
        # decode rows of a bf16 model use the grouped MFMA GEMM (small M, many
        # projections); prefill and other dtypes use library GEMMs
        grouped = decode and dt == torch.bfloat16 and self.use_grouped_gemm and M <= 1024
        for l in range(L):
            blk = self.blocks[l]
            att, ffn, pk = blk.att, blk.ffn, packs[l]
            kv, ax, fx = pool.kv[l], pool.att_x[l], pool.ffn_x[l]
            # residual (+ previous FFN) -> ln0/ln1 -> shift -> 6 lerps
            if l == 0:
                _lib.call("rwkv7_shift_mix", code, M, C, None, None, 0, 0, P(tokens), P(self.emb.weight),
                          cfg.vocab_size, P(pk.ln0[0]) if pk.ln0 else None, P(pk.ln0[1]) if pk.ln0 else None,
                          P(x_res), P(pk.ln1[0]), P(pk.ln1[1]), P(ax), S, P(row_slot), P(row_last), 7,
                          P(pk.mix7), P(mixes), st)
            else:
                _lib.call("rwkv7_shift_mix", code, M, C, P(x_mid), P(ffn_out), ffn_parts, ffn_stride, None, None,
                          0, None, None,
                          P(x_res), P(pk.ln1[0]), P(pk.ln1[1]), P(ax), S, P(row_slot), P(row_last), 7,
                          P(pk.mix7), P(mixes), st)
            xr, xk, xv, xw, xa, xg, _ = mixes.unbind(0)
            if grouped:
                # two grouped launches: r, k, v and the LoRA downs of the six
                # mixes (tanh on w, sigmoid on g as epilogues, into a [n][M][D]
                # buffer), then the four LoRA ups
                gp = pk.gp
                nl, D = pk.lora_down.shape[0], pk.lora_down.shape[2]
                key = (dev, M, nl, D)
                hbuf = self._lora_h.get(key)
                if hbuf is None:
                    hbuf = self._lora_h[key] = torch.zeros((nl, M, D), dtype=dt, device=dev)
                rkv = torch.empty((3, M, C), dtype=dt, device=dev)
                r, k, v = rkv.unbind(0)
                dn = [("w1", 0, 2), ("a1", 1, 0), ("g1", 2, 3)] + ([] if l == 0 else [("v1", 3, 0)])
                src = {"w1": xw, "a1": xa, "g1": xg, "v1": xv}
                probs = [(xr, gp["r"], r, 0), (xk, gp["k"], k, 0), (xv, gp["v"], v, 0)]
                probs += [(src[n], gp[n], hbuf[i, :, :gp[n].N], e) for n, i, e in dn]
                self._gemm_group(M, probs, st)
                up = torch.empty((nl, M, C), dtype=dt, device=dev)
                ups = [("w2", 0), ("a2", 1), ("g2", 2)] + ([] if l == 0 else [("v2", 3)])
                self._gemm_group(M, [(hbuf[i, :, :gp[n].K], gp[n], up[i], 0) for n, i in ups], st)
                wl, al, g = up[0], up[1], up[2]
                vl = up[3] if l > 0 else None
            else:
                # library GEMMs: r / k / v as three products on the [out][in]
                # weights (faster than one batched product over transposed
                # copies: 1.33 against 1.52 ms at 69,567 rows of a 1.5B layer), the
                # LoRA downs in one batched product (with tanh on w and sigmoid on
                # g between), the LoRA ups in one
                r = self._lin(xr, att.receptance.weight)
                k = self._lin(xk, att.key.weight)
                v = self._lin(xv, att.value.weight)
                nl = pk.lora_down.shape[0]
                h = torch.bmm(mixes[3:3 + nl], pk.lora_down)
                _lib.call("rwkv7_activation", code, 0, h[0].numel(), P(h[0]), st)
                _lib.call("rwkv7_activation", code, 1, h[2].numel(), P(h[2]), st)
                up = torch.bmm(h, pk.lora_up)
                wl, al, g = up[0], up[1], up[2]
                vl = up[3] if l > 0 else None
            o = torch.empty((M, C), dtype=dt, device=dev)
            if decode:
                _lib.call("rwkv7_tmix_decode", code, M, H, int(l == 0), P(r), P(k), P(v), P(wl), P(al),
                          P(vl), P(g), P(v_first), pk.tparams, P(kv), S, P(row_slot), P(o), st)
            else:
                _lib.call("rwkv7_tmix_prep", code, M, H, int(l == 0), P(r), P(k), P(v), P(wl), P(al),
                          P(vl), P(v_first), pk.tparams, ops_ptrs, st)
                wkv_ops.wkv7_prefill(kv, seq_slot, cu_seqlens, r, *ops.unbind(0), y=y)
                _lib.call("rwkv7_tmix_post", code, M, H, P(y), P(r), P(ops[1]), P(ops[2]), P(g),
                          pk.tparams, P(o), st)
            if grouped and self.use_grouped_output:
                # the output projection's K-range partials, summed by the next shift_mix
                att_out, att_parts = self._gemm_partials(M, o, pk.gp["o"], st)
                att_stride = M * C
            else:
                att_out, att_parts, att_stride = self._lin(o, att.output.weight), 0, 0
            # residual + attention -> ln2 -> FFN shift/lerp
            _lib.call("rwkv7_shift_mix", code, M, C, P(x_res), P(att_out), att_parts, att_stride, None, None, 0,
                      None, None,
                      P(x_mid), P(pk.ln2[0]), P(pk.ln2[1]), P(fx), S, P(row_slot), P(row_last), 1,
                      P(pk.mixk), P(xk_ffn), st)
            if grouped:
                # FFN key with relu^2 as its epilogue, then the value projection
                hk = torch.empty((M, pk.gp["fk"].N), dtype=dt, device=dev)
                self._gemm_group(M, [(xk_ffn[0], pk.gp["fk"], hk, 1)], st)
                # the value projection's K-range partials stay in the workspace;
                # the next row kernel (shift_mix / final_norm) sums them
                ffn_out, ffn_parts = self._gemm_partials(M, hk, pk.gp["fv"], st)
                ffn_stride = M * C
            else:
                hk = self._lin(xk_ffn[0], ffn.key.weight)
                _lib.call("rwkv7_activation", code, 2, hk.numel(), P(hk), st)
                ffn_out = self._lin(hk, ffn.value.weight)
                ffn_parts, ffn_stride = 0, 0
        n_out = M if logit_rows is None else (n_logit_rows if n_logit_rows is not None else logit_rows.numel())
        if n_out == 0:
            return None
        xo = torch.empty((n_out, C), dtype=dt, device=dev)
        _lib.call("rwkv7_final_norm", code, n_out, C, P(x_mid), P(ffn_out), ffn_parts, ffn_stride, P(logit_rows),
                  P(self._ln_out[0]), P(self._ln_out[1]), P(xo), st)
        if return_hidden:
            return xo
        return self._head_logits(xo)

    def _head_logits(self, xo: torch.Tensor) -> torch.Tensor:
        """logits = head(xo) (model.py:494-495): the library's head GEMM over the
        packed head for up to HeadPack.MAX_ROWS bf16 rows, a library GEMM otherwise."""
        hp = self._head_pack
        if (hp is not None and self.use_head_kernel and xo.shape[0] <= HeadPack.MAX_ROWS
                and xo.dtype == torch.bfloat16 and xo.stride(1) == 1):
            return hp.logits(xo)
        return self._lin(xo, self.head.weight)

    # -- reference-compatible entry points ------------------------------------

    @staticmethod
    def _meta_uniform(B: int, T: int, dev):
        idx = torch.arange(B * T, dtype=torch.int32)
        last = torch.full((B * T,), -1, dtype=torch.int32)
        last[0::T] = idx[T - 1::T]
        slot = (idx // T).to(torch.int32)
        cu = torch.arange(0, (B + 1) * T, T, dtype=torch.int32)
        return (slot.to(dev), last.to(dev), cu.to(dev), torch.arange(B, dtype=torch.int32).to(dev))

    @torch.no_grad()
    def forward_with_state(self, idx: torch.Tensor, states=None):
        """``(logits [B, T, V], new_states)``: the contract of ``model.py:468-497``.

        ``states`` is a list of per-layer dicts (``init_state``); the returned
        states are new float32 tensors (the inputs are not modified)."""
        self._check_device()
        if idx.ndim != 2:
            raise ValueError(f"idx must be [B, T], got {tuple(idx.shape)}")
        B, T = idx.shape
        if T == 0 or B == 0:
            raise ValueError("forward_with_state needs B > 0 and T > 0")
        dev = self.device
        cfg = self.config
        pool = StatePool(cfg, B, dev)
        if states is not None:
            if len(states) != cfg.n_layer:
                raise ValueError(f"expected {cfg.n_layer} layer states, got {len(states)}")
            for l, s in enumerate(states):
                pool.att_x[l].copy_(s["att_x_prev"].reshape(B, -1))
                pool.kv[l].copy_(s["att_kv"].reshape(pool.kv[l].shape))
                pool.ffn_x[l].copy_(s["ffn_x_prev"].reshape(B, -1))
        tokens = idx.to(device=dev, dtype=torch.int64).reshape(-1).contiguous()
        slot, last, cu, seq_slot = self._meta_uniform(B, T, dev)
        logits = self.forward_pooled(tokens, slot, last, pool, decode=(T == 1), cu_seqlens=cu,
                                     seq_slot=seq_slot)
        new_states = [{"att_x_prev": pool.att_x[l], "att_kv": pool.kv[l], "ffn_x_prev": pool.ffn_x[l]}
                      for l in range(cfg.n_layer)]
        return logits.view(B, T, -1), new_states

    @torch.no_grad()
    def forward_hidden(self, idx: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
        """ln_out hidden states ``[len(rows), n_embd]`` (model dtype) of a stateless
        forward over ``idx [B, T]`` from a zero state, for the flat positions
        ``rows`` (int32, b * T + t): the input of the head in ``forward``."""
        self._check_device()
        B, T = idx.shape
        pool = StatePool(self.config, B, self.device)
        tokens = idx.to(device=self.device, dtype=torch.int64).reshape(-1).contiguous()
        slot, last, cu, seq_slot = self._meta_uniform(B, T, self.device)
        rows = rows.to(device=self.device, dtype=torch.int32).contiguous()
        return self.forward_pooled(tokens, slot, last, pool, decode=(T == 1), cu_seqlens=cu, seq_slot=seq_slot,
                                   logit_rows=rows, n_logit_rows=rows.numel(), return_hidden=True)

    @torch.no_grad()
    def forward(self, idx: torch.Tensor, logits_to_keep: Optional[int] = None):
        """Stateless full-sequence logits (``model.py:435-466``), zero initial state."""
        self._check_device()
        B, T = idx.shape
        if T > self.config.ctx_len:
            raise AssertionError(f"Sequence length {T} exceeds max length {self.config.ctx_len}")
        pool = StatePool(self.config, B, self.device)
        tokens = idx.to(device=self.device, dtype=torch.int64).reshape(-1).contiguous()
        slot, last, cu, seq_slot = self._meta_uniform(B, T, self.device)
        keep = T if (logits_to_keep is None or logits_to_keep >= T) else logits_to_keep
        rows = (torch.arange(B, device=self.device)[:, None] * T
                + torch.arange(T - keep, T, device=self.device)[None, :]).reshape(-1).to(torch.int32)
        logits = self.forward_pooled(tokens, slot, last, pool, decode=(T == 1), cu_seqlens=cu,
                                     seq_slot=seq_slot, logit_rows=rows)
        return logits.view(B, keep, -1)


    @torch.no_grad()
    def generate(self, input_ids: Optional[torch.Tensor] = None, inputs: Optional[torch.Tensor] = None,
                 max_new_tokens: Optional[int] = None, max_length: Optional[int] = None,
                 min_length: Optional[int] = None, do_sample: bool = True, temperature: float = 1.0,
                 top_k: int = 0, top_p: float = 1.0, repetition_penalty: float = 1.0,
                 num_return_sequences: int = 1, eos_token_id=None, pad_token_id: Optional[int] = None,
                 token_ban: Optional[Sequence[int]] = None, return_dict_in_generate: bool = False,
                 output_scores: bool = False, initial_states=None, seed: Optional[int] = None, **kwargs):
        """Transformers-style generation with the semantics of the reference's
        ``GenerationMixin.generate`` (``rwkvtune/models/generation_mixin.py:33-225``):

        * ``input_ids`` ``[B, T]`` or ``[T]``; ``num_return_sequences`` repeats each
          row; ``max_new_tokens``, else ``max_length - T``, else 512 new tokens;
        * ``do_sample=False`` or ``temperature == 0`` is greedy argmax over the
          whole vocabulary (no id ban); otherwise temperature, ``token_ban`` (-inf),
          top-k and then, when 0 < top_p < 1, the nucleus keeping the crossing
          token (sampler rule 2); the repetition penalty counts every occurrence in
          the row's input and generated ids;
        * a row stops counting as unfinished when it emits an id of
          ``eos_token_id`` (an int or a list); generation ends when every row has,
          finished rows keep generating until then, as in the reference;
        * returns ``[B * num_return_sequences, T + generated]`` int64 (the input
          included), or ``{"sequences": ...}`` with ``return_dict_in_generate``.

        The prompt is prefilled in one ragged call and each new token is one
        pooled decode step; sampling is the device sampler (draws from its
        counter-based stream, keyed by ``seed``), so sampled tokens follow the
        reference's distribution, not ``torch.multinomial``'s stream.
        ``min_length``, ``pad_token_id`` and ``output_scores`` are accepted and,
        as in the reference, unused."""
        from .sampler import RULE_MIXIN, SamplerBuffers, TokenSampler, repetition_penalty_, sample_rows
        self._check_device()
        if input_ids is None:
            input_ids = inputs
        if input_ids is None:
            raise ValueError("Must provide input_ids or inputs parameter")
        if input_ids.dim() == 1:
            input_ids = input_ids.unsqueeze(0)
        B, T = input_ids.shape
        if T == 0:
            raise ValueError("generate needs at least one input token per row")
        if max_new_tokens is not None:
            n_new = int(max_new_tokens)
        elif max_length is not None:
            n_new = int(max_length) - T
        else:
            n_new = 512
        if eos_token_id is None:
            eos_token_id = getattr(self.config, "eos_token_id", None)
        eos = [] if eos_token_id is None else ([int(eos_token_id)] if isinstance(eos_token_id, int)
                                               else [int(e) for e in eos_token_id])
        if not do_sample:
            temperature, top_p, top_k = 1.0, 0.0, 0
        greedy = (not do_sample) or temperature == 0
        if num_return_sequences > 1:
            input_ids = input_ids.repeat_interleave(num_return_sequences, dim=0)
            B = B * num_return_sequences
        dev = self.device
        cfg = self.config
        ids = input_ids.to(device=dev, dtype=torch.int64)
        if n_new <= 0:
            return {"sequences": ids.clone()} if return_dict_in_generate else ids.clone()
        pool = StatePool(cfg, B, dev)
        if initial_states is not None:
            if len(initial_states) != cfg.n_layer:
                raise ValueError(f"expected {cfg.n_layer} layer states, got {len(initial_states)}")
            for l, st in enumerate(initial_states):
                pool.att_x[l].copy_(st["att_x_prev"].reshape(B, -1))
                pool.kv[l].copy_(st["att_kv"].reshape(pool.kv[l].shape))
                pool.ffn_x[l].copy_(st["ffn_x_prev"].reshape(B, -1))
        slot, last, cu, seq_slot = self._meta_uniform(B, T, dev)
        last_rows = (torch.arange(B, device=dev, dtype=torch.int32) * T + (T - 1)).contiguous()
        logits = self.forward_pooled(ids.reshape(-1).contiguous(), slot, last, pool, decode=(T == 1),
                                     cu_seqlens=cu, seq_slot=seq_slot, logit_rows=last_rows)
        width = T + n_new
        out = torch.zeros((B, width), dtype=torch.int64, device=dev)
        out[:, :T] = ids
        use_pen = repetition_penalty is not None and repetition_penalty != 1.0 and repetition_penalty > 0
        if use_pen:
            hist = torch.zeros((B, width), dtype=torch.int32, device=dev)
            hist[:, :T] = ids.to(torch.int32)
            h_start = torch.arange(B, dtype=torch.int64, device=dev) * width
            h_len = torch.empty(B, dtype=torch.int32, device=dev)
        ban = None
        if token_ban is not None and len(token_ban) > 0:
            ban = torch.tensor([int(t) for t in token_ban], dtype=torch.int64, device=dev)
        eos_t = torch.tensor(eos, dtype=torch.int64, device=dev) if eos else None
        unfinished = torch.ones(B, dtype=torch.bool, device=dev)
        buf = SamplerBuffers(B, dev)
        buf.set_uniform(0.0 if greedy else float(temperature), float(top_p), int(top_k))
        call_key = TokenSampler._next_key()
        buf.rng_key.copy_(torch.arange(B, dtype=torch.int64, device=dev) + (call_key << 24))
        if seed is None:
            seed = TokenSampler._seed
        row_slot = torch.arange(B, dtype=torch.int32, device=dev)
        tok = torch.empty(B, dtype=torch.int64, device=dev)
        lp = torch.empty(B, dtype=torch.float32, device=dev)
        done = n_new
        for step in range(n_new):
            lg = logits
            if use_pen:
                lg = lg.float()
                h_len.fill_(T + step)
                repetition_penalty_(lg, float(repetition_penalty), hist.view(-1), h_start, h_len)
            if ban is not None:
                lg = lg.clone() if lg is logits else lg
                lg[:, ban] = float("-inf")
            buf.rng_ctr.fill_(step)
            sample_rows(lg, buf, rule=RULE_MIXIN, max_valid_id=None, seed=seed, out_tok=tok, out_logp=lp)
            out[:, T + step] = tok
            if use_pen:
                hist[:, T + step] = tok.to(torch.int32)
            if eos_t is not None:
                unfinished &= ~torch.isin(tok, eos_t)
                if not bool(unfinished.any()):
                    done = step + 1
                    break
            if step + 1 < n_new:
                logits = self.forward_pooled(tok, row_slot, row_slot, pool, decode=True)
        seqs = out[:, :T + done]
        return {"sequences": seqs} if return_dict_in_generate else seqs


def build_model(config: RWKV7Config, dtype=torch.bfloat16, device="cuda", seed: int = 0) -> RWKV7Model:
    """Allocate a model on ``device`` in ``dtype`` and apply the seeded dense init."""
    with torch.device("meta"):
        m = RWKV7Model(config)
    m = m.to_empty(device=device)
    m = m.to(dtype)
    init_dense_(m, seed=seed, device=device)
    return m


# ---------------------------------------------------------------------------
# The caller's own model
# ---------------------------------------------------------------------------

_HIP_MODELS: "weakref.WeakKeyDictionary[nn.Module, RWKV7Model]" = weakref.WeakKeyDictionary()


def _config_of_params(params, src_config=None) -> RWKV7Config:
    """Architecture of a module carrying the reference's parameter names, read
    from the parameter shapes (``model.py:34-131, 281-302, 346-365, 421-433``)."""
    try:
        V, C = params["emb.weight"].shape
        L = 1 + max(int(n.split(".")[1]) for n in params if n.startswith("blocks."))
        dw = params["blocks.0.att.w1"].shape[1]
        dg = params["blocks.0.att.g1"].shape[1]
        dv = params["blocks.1.att.v1"].shape[1] if L > 1 else 0
    except (KeyError, ValueError) as e:
        raise ValueError(f"not an RWKV-7 module with the reference's parameter names ({e})") from None
    ctx = int(getattr(src_config, "ctx_len", 1024)) if src_config is not None else 1024
    return RWKV7Config(n_layer=L, n_embd=int(C), vocab_size=int(V), ctx_len=ctx, dim_att_lora=int(dw),
                       dim_gate_lora=int(dg), dim_mv_lora=int(dv))


def _lora_linears(module: nn.Module) -> dict:
    """Sub-modules wrapping an ``nn.Linear`` with a LoRA adapter the way the
    reference's ``LoraLinear`` does (``rwkvtune/peft/lora/layer.py:15-199``):
    ``base_layer``, ``lora_A [r, in]``, ``lora_B [out, r]``, ``scaling`` and the
    ``merged`` / ``disabled`` flags; the layer computes
    ``base_layer(x) + (x A^T) B^T * scaling`` unless merged or disabled."""
    out = {}
    for name, sub in module.named_modules():
        base = getattr(sub, "base_layer", None)
        if (isinstance(base, nn.Linear) and isinstance(getattr(sub, "lora_A", None), torch.Tensor)
                and isinstance(getattr(sub, "lora_B", None), torch.Tensor)):
            out[name] = sub
    return out


class _LoraMerge:
    """Keeps the wrapper's own weight of each LoRA-wrapped linear equal to
    ``W + scaling * B A`` (``W`` alone when the adapter is merged into ``W`` or
    disabled, ``layer.py:127-170``): recomputed, in float32 and rounded once to
    the weight's dtype, when the base weight, ``lora_A`` or ``lora_B`` changed
    (version or storage), or the scaling or flags did.  The result is copied into
    the same tensor, so the packs see a version bump and captured graphs keep
    their addresses."""

    def __init__(self):
        self.entries = []  # (lora module, destination parameter)
        self.keys = []

    def bind(self, entries):
        self.entries = list(entries)
        self.keys = [None] * len(self.entries)

    @staticmethod
    def _key(lm):
        W, A, B = lm.base_layer.weight, lm.lora_A, lm.lora_B
        return (W.data_ptr(), W._version, A.data_ptr(), A._version, B.data_ptr(), B._version,
                float(getattr(lm, "scaling", 1.0)), bool(getattr(lm, "merged", False)),
                bool(getattr(lm, "disabled", False)))

    @torch.no_grad()
    def __call__(self):
        for i, (lm, dst) in enumerate(self.entries):
            key = self._key(lm)
            if key == self.keys[i]:
                continue
            W = lm.base_layer.weight
            if key[-2] or key[-1]:
                dst.copy_(W)
            else:
                A, B = lm.lora_A.detach().float(), lm.lora_B.detach().float()
                dst.copy_(W.detach().float() + (B @ A) * key[-3])
            self.keys[i] = key


def _bind(m: RWKV7Model, module: nn.Module):
    """Point ``m``'s parameters at ``module``'s (the same ``Parameter`` objects),
    with a merged weight of its own for every LoRA-wrapped linear."""
    lora = _lora_linears(module)
    params = dict(module.named_parameters())
    ours = dict(m.named_parameters())
    expect = set(ours)
    for name in lora:
        expect.discard(name + ".weight")
        expect |= {name + ".base_layer.weight", name + ".lora_A", name + ".lora_B"}
    extra = sorted(set(params) - expect)
    missing = sorted(expect - set(params))
    if extra or missing:
        raise ValueError(f"{type(module).__name__} does not carry the RWKV-7 parameter set: "
                         f"missing {missing[:4]}, unexpected {extra[:4]}")
    devs = {p.device for p in params.values()}
    if len(devs) != 1:
        raise ValueError(f"parameters on several devices: {sorted(map(str, devs))}")
    merges = []
    for name, p in ours.items():
        owner, _, leaf = name.rpartition(".")
        if leaf == "weight" and owner in lora:
            lm = lora[owner]
            W = lm.base_layer.weight
            r = lm.lora_A.shape[0]
            if (tuple(W.shape) != tuple(p.shape) or tuple(lm.lora_A.shape) != (r, W.shape[1])
                    or tuple(lm.lora_B.shape) != (W.shape[0], r)):
                raise ValueError(f"{owner}: LoRA shapes W {tuple(W.shape)}, A {tuple(lm.lora_A.shape)}, "
                                 f"B {tuple(lm.lora_B.shape)} do not fit {tuple(p.shape)}")
            if lm.base_layer.bias is not None:
                raise ValueError(f"{owner}: the architecture's linears have no bias")
            own = p if getattr(p, "_lora_merged", False) and p.device == W.device and p.dtype == W.dtype \
                else None
            if own is None:
                own = nn.Parameter(torch.empty_like(W, memory_format=torch.contiguous_format), requires_grad=False)
                own._lora_merged = True
                m.get_submodule(owner)._parameters[leaf] = own
            merges.append((lm, own))
            continue
        src = params[name]
        if tuple(src.shape) != tuple(p.shape):
            raise ValueError(f"{name}: shape {tuple(src.shape)}, expected {tuple(p.shape)}")
        m.get_submodule(owner)._parameters[leaf] = src
    if merges:
        if m._pre_pack is None:
            m._pre_pack = _LoraMerge()
        m._pre_pack.bind(merges)
        m._pre_pack()
    else:
        m._pre_pack = None
    m._src_params = list(module.parameters())


def as_hip_model(module: nn.Module) -> RWKV7Model:
    """An ``RWKV7Model`` running ``module``'s own parameters on the HIP library.

    ``module`` is any ``nn.Module`` with the reference ``RWKV7Model``'s parameter
    names (``emb.weight``, ``blocks.{i}.att.receptance.weight``, ...) - the
    training model ``GRPOTrainer`` hands its rollout generator
    (``rwkvtune/training/grpo/lightning_module.py:708-750``), also after
    ``get_peft_model`` (``rwkvtune/training/grpo_trainer.py:381-393``) replaced
    some of its linears by LoRA layers (``base_layer`` + ``lora_A`` / ``lora_B``).
    The returned model registers the *same* ``Parameter`` objects (nothing is
    copied), so parameter updates are seen; a LoRA-wrapped linear gets a weight
    of its own, ``W + scaling * B A``, recomputed when ``W``, ``A`` or ``B``
    change.  Packed copies are refreshed when a parameter's version or storage
    changes.  One wrapper is kept per module; each call checks that ``module``
    still holds the same ``Parameter`` objects and re-binds the ones it replaced
    (``load_state_dict(assign=True)``, a LoRA layer added later).  An
    ``RWKV7Model`` is returned unchanged.  A module with parameters the
    architecture does not have is rejected."""
    if isinstance(module, RWKV7Model):
        return module
    hit = _HIP_MODELS.get(module)
    if hit is not None:
        cur = list(module.parameters())
        old = hit._src_params
        if len(cur) != len(old) or any(a is not b for a, b in zip(cur, old)):
            _bind(hit, module)
        return hit
    params = dict(module.named_parameters())
    lora = _lora_linears(module)
    if lora:
        for name in lora:
            params[name + ".weight"] = lora[name].base_layer.weight
    cfg = _config_of_params(params, getattr(module, "config", None))
    with torch.device("meta"):
        m = RWKV7Model(cfg)
    _bind(m, module)
    try:
        src_block0 = module.get_submodule("blocks.0")
    except AttributeError:
        src_block0 = None
    m.blocks[0].skip_ln0 = bool(getattr(src_block0, "skip_ln0", False))
    m.train(module.training)
    _HIP_MODELS[module] = m
    return m
