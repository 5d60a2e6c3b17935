"""Oracle for the batched MeanFlow FM/DiT head — TEST INFRASTRUCTURE ONLY.

This package is a CPU restatement (PyTorch, explicit casts, no autocast) of the
reference's DiT / MeanFlow solver / W8A8 linear math. It is the checker the HIP
path is compared against. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package
``nanovllm_dots_amd`` never does, and has no CPU fallback.

Modules:
  dit_ref    DiT forward (padded dense-mask form and varlen form), MeanFlow
             solve, FM mask / position builders, seeded weight init.
  int8_ref   W8A8 per-channel weight / per-token activation quantisation and
             the int32-accumulate linear.
  kvcache_ref  per-(timestep, layer) prefix K/V cache semantics for a
             MeanFlow solve (extend + active passes).
  paged_attn_ref  the LLM backbone's paged KV cache: store_kvcache and the
             varlen / paged attention (bottom-right causal, GQA) in float64.
"""
