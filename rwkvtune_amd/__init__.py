"""gfx950 (MI355X) implementation of rwkvtune's batched-generation hot path:
WKV7 decode / prefill kernels, the RWKV-7 stateful forward, device-side
sampling and a GPU slot-table rollout engine behind rwkvtune's own front ends,
the GRPO log-prob recompute that follows a rollout, and the WKV7 training
operator (forward + backward, with the infinite-context state variant).

Submodules import lazily so that loading the package needs neither a GPU nor
the built HIP library; every compute entry point raises if the library is
missing (there is no CPU fallback).
"""

__all__ = [
    "GRPOBatchGenerator", "SchedulerCore", "BatchGenerator", "GenerationConfig", "TokenSampler",
    "SamplingParams", "RWKV7Model", "RWKV7Config", "load_wkv_operator", "rwkv7_wkv",
    "selective_log_softmax", "compute_per_token_logps", "load_hip_operator_train", "rwkv7_wkv_infctx",
    "load_hip_operator_infctx",
]

_LAZY = {
    "GRPOBatchGenerator": ("grpo_batch_generator", "GRPOBatchGenerator"),
    "SchedulerCore": ("scheduler_core", "SchedulerCore"),
    "BatchGenerator": ("batch_generator", "BatchGenerator"),
    "GenerationConfig": ("batch_generator", "GenerationConfig"),
    "TokenSampler": ("sampler", "TokenSampler"),
    "SamplingParams": ("sampling_params", "SamplingParams"),
    "RWKV7Model": ("model", "RWKV7Model"),
    "RWKV7Config": ("model", "RWKV7Config"),
    "load_wkv_operator": ("operators", "load_wkv_operator"),
    "rwkv7_wkv": ("operators", "rwkv7_wkv"),
    "selective_log_softmax": ("grpo_utils", "selective_log_softmax"),
    "compute_per_token_logps": ("grpo_utils", "compute_per_token_logps"),
    "load_hip_operator_train": ("operators", "load_hip_operator_train"),
    "rwkv7_wkv_infctx": ("operators", "rwkv7_wkv_infctx"),
    "load_hip_operator_infctx": ("operators", "load_hip_operator_infctx"),
}


def __getattr__(name):
    if name in _LAZY:
        import importlib
        mod, attr = _LAZY[name]
        return getattr(importlib.import_module(f".{mod}", __name__), attr)
    raise AttributeError(name)
