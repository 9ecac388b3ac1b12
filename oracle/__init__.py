"""CPU oracle for the WKV7 decode / prefill / rollout path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``rwkvtune_amd`` imports this package:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker (or as the timed CPU baseline),
never as the thing measured or shipped.

Contents
--------
``wkv7``      torch-CPU restatement of the reference's WKV7 recurrence
              (``rwkvtune/models/rwkv7/operators/wkv_cpu.py:9-76`` and the
              per-row order of ``operators/cuda/wkv7s.cu:22-53``).
``cref``      ctypes binding of ``wkv7_ref.c``: an independent fp64 scalar
              restatement of the same recurrence in C.
``model``     torch-CPU restatement of ``RWKV7Model.forward_with_state``
              (``rwkvtune/models/rwkv7/model.py:174-520``).
``sampler``   restatement of ``TokenSampler`` (``rwkvtune/inference/core.py:16-236``).
``logprob``   restatement of the GRPO log-prob recompute
              (``rwkvtune/training/grpo/utils.py:13-103``,
              ``grpo/lightning_module.py:1810-1964``).
``rollout``   restatement of the GRPO rollout loop
              (``rwkvtune/inference/grpo_batch_generator.py:115-748``), used as the
              CPU baseline.

Pinning (what each function is checked against, besides itself) is listed in the
header of each module and exercised in ``tests/test_oracle_*.py``.
"""
