"""``RWKV7Model.generate`` (the reference's ``GenerationMixin.generate``,
``rwkvtune/models/generation_mixin.py:33-225``) and the trainer-model drop-in of
the rollout front ends (``rwkvtune/training/grpo/lightning_module.py:708-787``).

* greedy ``generate`` (do_sample=False) token ids equal the CPU oracle's greedy
  decode over the whole vocabulary (``oracle.model.greedy_generate`` with no
  ban), float32 toy model; num_return_sequences repeats rows; an EOS list ends
  generation when every row has emitted one (rows that finished earlier keep
  generating, as in the reference); max_length; dict return.
* ``GRPOBatchGenerator(model=<plain nn.Module with the reference's parameter
  names>)``: greedy paths equal those of a freshly built model carrying the same
  weights, before and after a ``torch.optim.SGD`` step that updates the
  parameters in place between two ``generate`` calls (no ``invalidate()``), for
  float32 (library-GEMM decode) and bf16 (packed-weight decode GEMM) models.
"""

import pytest
import torch
import torch.nn as nn

from oracle import model as om
from rwkvtune_amd.grpo_batch_generator import GRPOBatchGenerator
from rwkvtune_amd.model import RWKV7Config, RWKV7Model, as_hip_model, build_model

pytestmark = pytest.mark.gpu

V = 1000


def tiny(dtype, seed):
    cfg = RWKV7Config(n_layer=2, n_embd=256, vocab_size=V, dim_att_lora=32, dim_gate_lora=64, dim_mv_lora=32)
    return build_model(cfg, dtype=dtype, device="cuda", seed=seed)


def test_generate_greedy_matches_oracle(gpu_device):
    print("[case] generate greedy vs oracle", flush=True)
    m = tiny(torch.float32, 41)
    sd = om.cast_state_dict(m.state_dict(), torch.float32)
    g = torch.Generator().manual_seed(42)
    prompts = torch.randint(0, V, (3, 17), generator=g)
    out = m.generate(prompts.to(gpu_device), max_new_tokens=12, do_sample=False)
    ref, _ = om.greedy_generate(sd, prompts, 12, dtype=torch.float32, max_valid_id=None)
    assert out.shape == (3, 17 + 12)
    assert torch.equal(out[:, :17].cpu(), prompts)
    assert torch.equal(out[:, 17:].cpu(), ref)
    # 1-D input, max_length, dict return, num_return_sequences
    d = m.generate(prompts[0].to(gpu_device), max_length=17 + 5, do_sample=False, return_dict_in_generate=True,
                   num_return_sequences=2)
    seq = d["sequences"].cpu()
    assert seq.shape == (2, 22)
    assert torch.equal(seq[0], seq[1]) and torch.equal(seq[0, 17:], ref[0, :5])


def test_generate_eos_stops_when_every_row_finished(gpu_device):
    print("[case] generate EOS", flush=True)
    m = tiny(torch.float32, 43)
    sd = om.cast_state_dict(m.state_dict(), torch.float32)
    prompts = torch.randint(0, V, (2, 9), generator=torch.Generator().manual_seed(44))
    ref, _ = om.greedy_generate(sd, prompts, 10, dtype=torch.float32, max_valid_id=None)
    # EOS ids: row 0's 3rd token and row 1's 6th token (unless they appear earlier)
    eos = [int(ref[0, 2]), int(ref[1, 5])]
    ends = []
    for r in range(2):
        hit = [i for i in range(10) if int(ref[r, i]) in eos]
        ends.append(hit[0] + 1 if hit else 10)
    n = max(ends)
    out = m.generate(prompts.to(gpu_device), max_new_tokens=10, do_sample=False, eos_token_id=eos).cpu()
    assert out.shape == (2, 9 + n)
    assert torch.equal(out[:, 9:], ref[:, :n])


def test_generate_sampled_rows_are_reproducible_and_valid(gpu_device):
    print("[case] generate sampled", flush=True)
    m = tiny(torch.bfloat16, 45)
    prompts = torch.randint(0, V, (4, 8), generator=torch.Generator().manual_seed(46)).to(gpu_device)
    kw = dict(max_new_tokens=16, temperature=0.9, top_p=0.8, top_k=50, repetition_penalty=1.3, token_ban=[3, 4],
              seed=7)
    a = m.generate(prompts, **kw)
    b = m.generate(prompts, **kw)
    assert a.shape == (4, 24)
    new = a[:, 8:]
    assert bool(((new >= 0) & (new < V)).all())
    assert not bool(torch.isin(new, torch.tensor([3, 4], device=gpu_device)).any())
    # different call keys draw different streams; equal shape and validity hold for both
    assert b.shape == a.shape


def _plain_module(model):
    """An nn.Module tree with the reference model's parameter names and nothing
    else: not an RWKV7Model, no forward."""
    root = nn.Module()
    for name, t in model.state_dict().items():
        mod = root
        parts = name.split(".")
        for q in parts[:-1]:
            if not hasattr(mod, q):
                mod.add_module(q, nn.Module())
            mod = getattr(mod, q)
        mod.register_parameter(parts[-1], nn.Parameter(t.detach().clone()))
    return root


class _Tok:
    eos_token_id = None

    def __init__(self):
        self.idx2token = {i: str(i).encode() for i in range(V - 3)}

    def decode(self, ids):
        return " ".join(str(i) for i in ids)


def _fresh(src, dtype):
    m = tiny(dtype, 0)
    m.load_state_dict({k: v.detach().clone() for k, v in src.state_dict().items()})
    return m


def _greedy_paths(model, prompts):
    gen = GRPOBatchGenerator(model, _Tok(), chunk_size=16, max_decode_batch_size=4, verbose=False)
    out = gen.generate(prompts, 10, num_generations=2, temperature=0.0, top_p=1.0)
    ids, masks = out["completion_ids"].cpu(), out["masks"].cpu()
    return [ids[q, :int(masks[q].sum())].tolist() for q in range(ids.shape[0])]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_trainer_model_dropin_follows_optimizer_steps(gpu_device, dtype):
    print(f"[case] trainer-model drop-in {dtype}", flush=True)
    src = _plain_module(tiny(dtype, 47))
    assert not isinstance(src, RWKV7Model)
    g = torch.Generator().manual_seed(48)
    prompts = [torch.randint(0, V - 3, (n,), generator=g).tolist() for n in (5, 23, 11)]
    gen = GRPOBatchGenerator(src, _Tok(), chunk_size=16, max_decode_batch_size=4, verbose=False)
    assert gen.model is src and as_hip_model(src) is gen._hip

    def run():
        out = gen.generate(prompts, 10, num_generations=2, temperature=0.0, top_p=1.0)
        ids, masks = out["completion_ids"].cpu(), out["masks"].cpu()
        return [ids[q, :int(masks[q].sum())].tolist() for q in range(ids.shape[0])]

    before = run()
    assert before == _greedy_paths(_fresh(src, dtype), prompts)
    # one optimizer step on every parameter, in place, as a trainer makes it
    opt = torch.optim.SGD(src.parameters(), lr=0.5)
    for p in src.parameters():
        p.grad = torch.randn(p.shape, generator=torch.Generator(device=p.device).manual_seed(p.numel() % 997),
                             device=p.device).to(p.dtype) * p.detach().float().std().clamp_min(1e-3).to(p.dtype)
    opt.step()
    after = run()
    assert after == _greedy_paths(_fresh(src, dtype), prompts)
    assert after != before


def test_storage_swap_and_parameter_replacement_rebuild_graphs(gpu_device):
    """A parameter whose storage is swapped (``p.data = ...``, as FSDP / ZeRO-3
    gathers do) between two ``generate`` calls makes the captured decode graphs
    stale (they read the embedding and the head in place): the pack generation
    moves, the graphs are rebuilt, and the paths equal a fresh model's.  The same
    holds when the module's ``Parameter`` objects are replaced
    (``load_state_dict(assign=True)``): the wrapper re-binds to the new ones."""
    print("[case] storage swap / parameter replacement", flush=True)
    dtype = torch.bfloat16
    src = _plain_module(tiny(dtype, 51))
    g = torch.Generator().manual_seed(52)
    prompts = [torch.randint(0, V - 3, (n,), generator=g).tolist() for n in (7, 19)]
    gen = GRPOBatchGenerator(src, _Tok(), chunk_size=16, max_decode_batch_size=4, verbose=False)

    def run():
        out = gen.generate(prompts, 10, num_generations=2, temperature=0.0, top_p=1.0)
        ids, masks = out["completion_ids"].cpu(), out["masks"].cpu()
        return [ids[q, :int(masks[q].sum())].tolist() for q in range(ids.shape[0])]

    before = run()
    gen0 = gen._hip._packs_gen
    gw = torch.Generator(device=gpu_device).manual_seed(53)
    with torch.no_grad():
        for name in ("emb.weight", "head.weight", "blocks.1.ffn.key.weight"):
            p = src.get_parameter(name)
            p.data = (p.data.float() + 0.3 * torch.randn(p.shape, generator=gw, device=gpu_device)
                      * p.data.float().std()).to(dtype)
    after = run()
    assert gen._hip._packs_gen > gen0
    assert after == _greedy_paths(_fresh(src, dtype), prompts)
    assert after != before
    # new Parameter objects: the wrapper follows them
    hip = gen._hip
    sd = {k: (v.detach().float() * 1.25).to(dtype) for k, v in src.state_dict().items()}
    src.load_state_dict(sd, assign=True)
    again = run()
    assert gen._hip is hip
    assert again == _greedy_paths(_fresh(src, dtype), prompts)


class _LoraLinear(nn.Module):
    """A linear wrapped with a LoRA adapter under the attribute names of the
    reference's ``LoraLinear`` (``rwkvtune/peft/lora/layer.py:15-199``)."""

    def __init__(self, weight, r, alpha):
        super().__init__()
        out_f, in_f = weight.shape
        self.base_layer = nn.Linear(in_f, out_f, bias=False, device=weight.device, dtype=weight.dtype)
        with torch.no_grad():
            self.base_layer.weight.copy_(weight)
        self.base_layer.weight.requires_grad_(False)
        self.r, self.scaling = r, alpha / r
        g = torch.Generator(device=weight.device).manual_seed(out_f * 31 + in_f)
        self.lora_A = nn.Parameter((torch.rand(r, in_f, generator=g, device=weight.device) - 0.5)
                                   .mul(2 / in_f ** 0.5).to(weight.dtype))
        self.lora_B = nn.Parameter(torch.zeros(out_f, r, device=weight.device, dtype=weight.dtype))
        self.merged = False
        self.disabled = False


LORA_TARGETS = ("att.receptance", "att.key", "att.value", "att.output", "ffn.key", "ffn.value")


def _merged_state(src, dtype):
    """The plain model a LoRA-wrapped module computes: W + scaling * B A per
    wrapped linear (float32, rounded once)."""
    sd = {}
    for name, mod in src.named_modules():
        if isinstance(mod, _LoraLinear):
            W = mod.base_layer.weight.detach().float()
            if not (mod.merged or mod.disabled):
                W = W + (mod.lora_B.detach().float() @ mod.lora_A.detach().float()) * mod.scaling
            sd[name + ".weight"] = W.to(dtype)
    for name, p in src.named_parameters():
        if ".base_layer." not in name and not name.endswith(("lora_A", "lora_B")):
            sd[name] = p.detach()
    return sd


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_trainer_model_dropin_with_lora(gpu_device, dtype):
    """The call site in LoRA mode (``GRPOTrainer`` wraps its model with
    ``get_peft_model``, ``rwkvtune/training/grpo_trainer.py:381-393``, and hands it
    to the generator, ``grpo/lightning_module.py:708-750``): greedy paths equal a
    fresh model built from the merged weights, before and after an optimizer
    step on ``lora_A`` / ``lora_B`` only, and with the adapters disabled."""
    print(f"[case] LoRA drop-in {dtype}", flush=True)
    src = _plain_module(tiny(dtype, 55))
    for name, mod in list(src.named_modules()):
        if name.endswith(LORA_TARGETS) and name.count(".") == 3:
            parent = src.get_submodule(name.rpartition(".")[0])
            setattr(parent, name.rpartition(".")[2], _LoraLinear(mod.weight.detach(), 16, 32))
    lora_params = [p for n, p in src.named_parameters() if n.endswith(("lora_A", "lora_B"))]
    assert len(lora_params) == 2 * 6 * 2
    g = torch.Generator().manual_seed(56)
    prompts = [torch.randint(0, V - 3, (n,), generator=g).tolist() for n in (6, 21, 13)]
    gen = GRPOBatchGenerator(src, _Tok(), chunk_size=16, max_decode_batch_size=4, verbose=False)

    def run():
        out = gen.generate(prompts, 10, num_generations=2, temperature=0.0, top_p=1.0)
        ids, masks = out["completion_ids"].cpu(), out["masks"].cpu()
        return [ids[q, :int(masks[q].sum())].tolist() for q in range(ids.shape[0])]

    def fresh():
        m = tiny(dtype, 0)
        m.load_state_dict({k: v.clone() for k, v in _merged_state(src, dtype).items()})
        return m

    before = run()  # B = 0: the base model
    assert before == _greedy_paths(fresh(), prompts)
    opt = torch.optim.SGD(lora_params, lr=1.0)
    for i, p in enumerate(lora_params):
        gg = torch.Generator(device=p.device).manual_seed(100 + i)
        p.grad = (torch.randn(p.shape, generator=gg, device=p.device) * 0.05).to(p.dtype)
    opt.step()
    after = run()
    assert after == _greedy_paths(fresh(), prompts)
    assert after != before
    for mod in src.modules():
        if isinstance(mod, _LoraLinear):
            mod.disabled = True
    assert run() == before
