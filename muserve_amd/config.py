"""Constants of the KV-cache path, mirroring muserve/config.py:5-9,20-24,27,36-37.

Only the values the cache layer reads are kept. The pool classes take sizes
and dtypes as constructor arguments; these are their defaults.
"""

NUM_LAYERS = 60          # muserve/config.py:5 (15 attention + 45 GDN layers)
NUM_KV_HEADS = 2         # muserve/config.py:8
HEAD_DIM = 256           # muserve/config.py:9

GDN_NUM_K_HEADS = 16     # muserve/config.py:20
GDN_NUM_V_HEADS = 64     # muserve/config.py:21
GDN_KEY_DIM = 128        # muserve/config.py:22
GDN_VALUE_DIM = 128      # muserve/config.py:23
GDN_CONV_KERNEL = 4      # muserve/config.py:24

TP_SIZE = 8              # muserve/config.py:27
MAX_DECODE_BATCH = 256   # muserve/config.py:33

KV_PAGE_SIZE = 16        # muserve/config.py:36
KV_DTYPE = "float16"     # muserve/config.py:37

# Attention layers of the 60-layer hybrid stack (every fourth layer),
# muserve/memory/kv_cache.py:20.
ATTN_LAYER_INDICES = [3, 7, 11, 15, 19, 23, 27, 31, 35, 39, 43, 47, 51, 55, 59]

MAX_SEQ_LEN = 262144            # muserve/config.py:10
CHUNKED_PREFILL_SIZE = 4096     # muserve/config.py:40
