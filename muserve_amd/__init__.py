"""MI355X-native KV-cache hot path for muserve.

Drop-in modules with the reference's class names and signatures:

* ``muserve_amd.kv_cache``        -> ``PagedKVCache``, ``SequenceKVState``
                                     (muserve/kv_cache.py), plus the batched
                                     ``BlockTables`` decode helper
* ``muserve_amd.memory.kv_cache`` -> ``KVCache`` (muserve/memory/kv_cache.py)
* ``muserve_amd.model.prefix_cache`` -> ``PrefixCache``
                                     (muserve/model/prefix_cache.py)
* ``muserve_amd.state_pool``      -> ``StatePool`` for GDN recurrent/conv states
* ``muserve_amd.block_manager``   -> ``BlockManager`` (refcounts, copy-on-write,
                                     prefix-hash table, LRU eviction)
* ``muserve_amd.scheduler``       -> ``ContinuousBatchScheduler``,
                                     ``InferenceRequest`` (muserve/scheduler.py),
                                     plus the paged step plan (chunked prefill)

All device work runs in hand-written gfx950 HIP kernels in libmuserve_kv.so
(C ABI: include/mkv.h), reached through ``muserve_amd._lib``. There is no CPU
or torch fallback for the kernels: without the built library, or with tensors
off the GPU, the calls raise.
"""

__version__ = "0.1.0"
