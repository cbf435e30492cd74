"""MI355X-native ragged paged-attention path for M*.

Batch packing, paged KV append and paged GQA attention (split-KV decode and
ragged MFMA prefill) as hand-written gfx950 HIP kernels behind a C ABI
(``include/mstar_amd.h``), with Python host classes that keep the
interfaces M*'s engine calls:

* :mod:`mstar_amd.paged_attention` — ``FlashInferPrefillWrapper`` /
  ``FlashInferDecodeWrapper`` plan()/run()/set_kv_cache() surface.
* :mod:`mstar_amd.cache_manager` — ``BatchedCacheManager`` (GPU packing).
* :mod:`mstar_amd.kv_store` — FIFO page allocator, request state, device block table.
"""

__version__ = "0.1.0"
