"""CPU oracle for the KV-cache path — TEST INFRASTRUCTURE ONLY.

Restatements of the reference's semantics (muserve/kv_cache.py,
muserve/memory/kv_cache.py, muserve/model/prefix_cache.py,
muserve/model/qwen35_layer_v2.py) in torch-CPU, numpy, hashlib and
collections.OrderedDict, each function citing the reference lines it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or the timed CPU baseline;
the product (muserve_amd) never imports it and has no CPU fallback.

Pinning (what checks each function beyond its own restatement):
  paged.PoolModel alloc/free      known answers of muserve/scripts/test_kv_cache.py:25-55
  paged.SeqModel / page_table     known answers of muserve/scripts/test_kv_cache.py:87-111
  paged.write_kv / gather_*       exact round trip (test_kv_cache.py:58-84) and a
                                  per-position pure-Python brute force on small cases
  fp8.fast_fp8_quantize           torch's e4m3fn cast vs fp8.e4m3fn_nearest (brute-force
                                  nearest-value search, ties to even) + hand-derived
                                  special values; scale vs closed forms
  fp8.dequant                     exact fp8 decode table vs the OFP8 definition
  sha.*                           FIPS 180-4 example vectors; per-page hashes vs
                                  hashing each prefix from scratch
  lru.PrefixCacheModel            scripted traces with hand-derived eviction order
  blocks.BlockManagerModel        invariants (refcounts = holders; free+used+cached = P;
                                  no eviction of referenced pages) and an independent
                                  timestamp-LRU brute force (blocks.TimestampLRUModel)
                                  on small traces
  state.gather/scatter            round trip and index_select/index_copy_ identities
  attention.decode_attention      torch scaled_dot_product_attention (float64) on the
                                  gathered K/V; closed forms (one token, constant V, equal
                                  keys, one dominant key); invariance when the pool's
                                  pages move; the reference's bf16 contiguous formula
                                  (attention.reference_bf16) within bf16 rounding
"""
