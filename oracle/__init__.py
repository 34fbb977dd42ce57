"""CPU oracle for the Tinytron decode step (TEST INFRASTRUCTURE ONLY).

This package restates, on the CPU, the algorithm of the reference's inference
decode path (liangyuwang/Tinytron):

* ``tinytron/model/modules/attn.py:13-63``   rope_impl (HF half-split RoPE)
* ``tinytron/model/modules/attn.py:66-83``   gqa_impl (K/V head expansion)
* ``tinytron/model/modules/attn.py:86-95``   build_cache_causal_mask
* ``tinytron/inference/cache.py:11-97``      LayerPagedKVCache / PagedKVCache
* ``tinytron/model/modules/attn.py:420-423`` F.scaled_dot_product_attention call
* ``tinytron/inference/sampler.py:6-48``     filter_logits / sample_next_token
* ``tinytron/inference/engine.py:144-261``   InferenceEngine.generate loop

plus the pieces this build adds on top of the reference (page table, ragged
per-sequence lengths, fp8-e4m3fn cache with per-token-per-head scales).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker or the timed CPU
baseline. The product (``tinytron_amd``) never imports it: the GPU path has
no CPU fallback.

Modules
-------
numerics   bf16 / fp8-e4m3fn rounding emulation in numpy (pinned against
           torch's casts, exhaustively for the 256 fp8 codes).
rope       cos/sin table and per-op-rounded RoPE (pinned against the fp64
           rotation closed form and against torch's own bf16 ops).
kvcache    slot / page / physical-page arithmetic, append, gather, fp8
           quantize-on-append (pinned by closed forms and brute force).
attention  fp64 textbook decode attention and the split-K (m, l, o) merge
           (pinned by special cases and by torch's SDPA in fp64).
sampler    filter_logits / greedy restated (pinned: top_k=1 == argmax).
ref_path   torch-CPU restatement of the reference op sequence, used as the
           timed CPU baseline and for end-to-end token parity.
"""
