// mkv_hash.hip — per-page SHA-256 prefix hashes for the prefix cache (gfx950).
//
// The key of a prefix is the first 8 bytes of SHA-256 over its token ids as
// little-endian integers (muserve/model/prefix_cache.py:31-34). A page is 16
// tokens, i.e. 128 bytes of int64 ids = exactly two SHA-256 blocks, so the
// hash of "the prefix ending at page i" is the running SHA-256 state after
// page i, finalised with one constant padding block. A request's pages form a
// dependent chain; requests are independent, so one lane walks one request
// and a launch covers a whole batch of requests. The work is integer ALU and
// latency bound (two chained compressions per page plus one to finalise),
// not HBM bound.
#include "mkv_device.h"

namespace mkv {
namespace {

__global__ __launch_bounds__(kThreads) void block_hash_kernel(const uint8_t* tokens,
                                                             const int64_t* tok_off,
                                                             const int64_t* page_off,
                                                             int32_t num_requests,
                                                             int32_t token_bytes, uint64_t* out,
                                                             int32_t* err) {
  const int r = blockIdx.x * kThreads + threadIdx.x;
  if (r >= num_requests) return;
  const int64_t t0 = tok_off[r], t1 = tok_off[r + 1];
  const int64_t o0 = page_off[r], o1 = page_off[r + 1];
  if (t1 < t0) {
    raise_err(err, MKV_DEVERR_TABLE);
    return;
  }
  const int64_t pages = (t1 - t0) / 16;
  if (o1 - o0 != pages) {  // the caller's page offsets disagree with the token counts
    raise_err(err, MKV_DEVERR_TABLE);
    return;
  }
  const uint32_t* p = reinterpret_cast<const uint32_t*>(tokens + t0 * token_bytes);
  const int blocks_per_page = token_bytes * 16 / 64;  // 2 for int64 ids, 1 for int32
  const uint64_t page_bytes = (uint64_t)token_bytes * 16u;
  Sha256 s;
  sha256_init(s);
  for (int64_t i = 0; i < pages; ++i) {
    for (int k = 0; k < blocks_per_page; ++k) {
      uint32_t w[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) w[j] = bswap32(p[j]);
      sha256_compress(s, w);
      p += 16;
    }
    out[o0 + i] = sha256_final_aligned_u64(s, (uint64_t)(i + 1) * page_bytes);
  }
}

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int mkv_block_hash_sha256(const void* tokens, const int64_t* tok_offsets,
                                     const int64_t* page_offsets, int32_t num_requests,
                                     int32_t token_bytes, uint64_t* out, int32_t* err,
                                     void* stream) {
  clear_error();
  MKV_REQUIRE(num_requests >= 0, MKV_E_INVALID, "mkv_block_hash_sha256: negative count");
  MKV_REQUIRE(token_bytes == 8 || token_bytes == 4, MKV_E_UNSUPPORTED,
              "mkv_block_hash_sha256: token_bytes %d unsupported (4 or 8)", token_bytes);
  if (num_requests == 0) return MKV_OK;
  MKV_REQUIRE(tokens && tok_offsets && page_offsets && out && err, MKV_E_INVALID,
              "mkv_block_hash_sha256: null pointer");
  MKV_REQUIRE(((uintptr_t)tokens & 3) == 0, MKV_E_ALIGN,
              "mkv_block_hash_sha256: tokens must be 4-byte aligned");
  hipLaunchKernelGGL(block_hash_kernel, dim3((num_requests + kThreads - 1) / kThreads),
                     dim3(kThreads), 0, as_stream(stream), (const uint8_t*)tokens, tok_offsets,
                     page_offsets, num_requests, token_bytes, out, err);
  return check_launch("mkv_block_hash_sha256");
}
