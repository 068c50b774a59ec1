"""PagedKVCache() with no page count: the pool is sized from the device's free
memory as muserve/kv_cache.py:60-73 sizes it (90 % of mem_get_info's free
bytes over the bytes of one page in all 60 layers, at least 1024 pages), with
the element size taken from the dtype and, for fp8, the per-token scale
counted. The hand-worked arithmetic is pinned on the CPU
(tests/test_host_paged.py::test_estimate_pages_closed_form); here the real
device query sizes a real pool, which must then work at its far end, where
byte offsets are far past 2^32."""
import pytest
import torch

from muserve_amd.config import HEAD_DIM, KV_PAGE_SIZE, NUM_LAYERS
from muserve_amd.kv_cache import PagedKVCache
from tests.gpu_util import DEV, bits16, case

pytestmark = pytest.mark.gpu

ELEM_BYTES = {None: 2, torch.float16: 2, torch.bfloat16: 2, torch.float8_e4m3fn: 1}


@pytest.mark.parametrize("dtype", [None, torch.bfloat16, torch.float8_e4m3fn])
def test_default_sized_pool(dtype):
    case(f"PagedKVCache() sized from free HBM, dtype {dtype or 'default (fp16)'}")
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    free = torch.cuda.mem_get_info(DEV)[0]
    per_token = HEAD_DIM * ELEM_BYTES[dtype] + (4 if dtype == torch.float8_e4m3fn else 0)
    page_bytes = NUM_LAYERS * 2 * KV_PAGE_SIZE * 1 * per_token
    want = max(1024, (free - int(free * 0.10)) // page_bytes)
    cache = PagedKVCache(device=DEV, dtype=dtype, verbose=False)
    try:
        assert cache.num_pages == want
        assert cache.dtype == (dtype or torch.float16)
        assert tuple(cache.cache.shape) == (NUM_LAYERS, 2, want, KV_PAGE_SIZE, 1, HEAD_DIM)
        # the last page of the last layer: the farthest bytes of the pool
        last = cache.num_pages - 1
        layer = NUM_LAYERS - 1
        g = torch.Generator().manual_seed(5)
        k = torch.randn(16, 1, HEAD_DIM, generator=g).bfloat16()
        if cache.dtype == torch.float16:
            k = k.half()
        slots = torch.arange(last * 16, last * 16 + 16, dtype=torch.int64, device=DEV)
        cache.append(slots, k.to(DEV), (-k).to(DEV), layer=layer)
        bt = torch.tensor([[last]], dtype=torch.int32, device=DEV)
        sl = torch.tensor([16], dtype=torch.int32, device=DEV)
        ko, vo = cache.gather(layer, bt, sl, out_len=16)
        cache.check_errors()
        if cache.dtype == torch.float8_e4m3fn:
            # quantised on append: the dequantised rows match the pool's own
            # codes and scales, and the signs of K and -K agree
            codes = cache.cache[layer, 0, last].float().cpu()
            scale = cache.scales[layer, 0, last].cpu()
            assert torch.equal(bits16(ko[0]), (codes * scale[..., None]).bfloat16().view(torch.int16))
            assert torch.equal(bits16(vo[0]), bits16(-ko[0]))
        else:
            assert torch.equal(bits16(ko[0]), k.view(torch.int16))
            assert torch.equal(bits16(vo[0]), (-k).view(torch.int16))
    finally:
        del cache
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
