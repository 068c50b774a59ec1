"""The path's constants against the reference's (muserve/config.py:5-9,20-24,
33,36-37,40; attention layer indices muserve/memory/kv_cache.py:20)."""
from muserve_amd import config as C


def test_layer_split_of_the_hybrid_stack():
    assert C.NUM_LAYERS == 60
    assert C.ATTN_LAYER_INDICES == [l for l in range(C.NUM_LAYERS) if l % 4 == 3]
    assert len(C.ATTN_LAYER_INDICES) == 15
    assert C.NUM_LAYERS - len(C.ATTN_LAYER_INDICES) == 45  # GDN layers


def test_pool_geometry():
    assert C.KV_PAGE_SIZE == 16
    assert C.HEAD_DIM == 256
    assert C.KV_DTYPE == "float16"
    assert max(1, C.NUM_KV_HEADS // C.TP_SIZE) == 1  # KV heads per rank in the pool
    assert C.MAX_DECODE_BATCH == 256
    assert C.CHUNKED_PREFILL_SIZE == 4096


def test_gdn_state_geometry():
    assert (C.GDN_NUM_K_HEADS, C.GDN_NUM_V_HEADS) == (16, 64)
    assert (C.GDN_KEY_DIM, C.GDN_VALUE_DIM, C.GDN_CONV_KERNEL) == (128, 128, 4)
    assert C.GDN_NUM_V_HEADS // C.TP_SIZE == 8  # recurrent state heads per rank
