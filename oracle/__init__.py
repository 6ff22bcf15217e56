"""Oracle: CPU restatements of the reference's continuous-batching attention path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or as the timed CPU baseline.  The product package
(``nano_vllm_ascend_amd``) never imports it and has no CPU fallback.

Modules
-------
attention_ref      fp32 torch-CPU paged decode, dense and paged causal varlen
                   prefill, KV store, per-head RMSNorm + rotate-half RoPE.
block_manager_ref  plain-Python restatement of the reference BlockManager,
                   including the per-token slot loop the GPU packing replaces.
qwen3_ref          torch restatement of the reference Qwen3 forward (fp32, or
                   bf16 at the reference's rounding points) for greedy-token
                   and logits parity of the whole model.

How each function is pinned (checked against something other than itself) is
listed in the module docstrings and exercised by ``tests/test_oracle.py``.
The reference publishes no numeric vectors for attention, RMSNorm or RoPE
(its arithmetic lives in closed torch_npu/CANN operators), so those are pinned
by library routines (torch SDPA, HF transformers' Qwen3 layers), brute force on
tiny inputs and invariants; the block manager is pinned by the reference's own
known-answer tests and by golden traces written from the reference source.
"""
