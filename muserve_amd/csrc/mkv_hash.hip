// mkv_hash.hip — per-page SHA-256 prefix hashes for the prefix cache (gfx950).
//
// The key of a prefix is the first 8 bytes of SHA-256 over its token ids as
// little-endian integers (muserve/model/prefix_cache.py:31-34). A page is 16
// tokens, i.e. 128 bytes of int64 ids = exactly two SHA-256 blocks (one for
// int32 ids), so the hash of "the prefix ending at page i" is the running
// SHA-256 state after page i, finalised with one constant-length padding
// block. A request's pages form a dependent chain of compressions, and the
// kernel is bound by instruction issue along that chain (a compression is
// ~1,500 VALU instructions), not by HBM.
//
// Two adjacent lanes share a request: the even lane absorbs the token blocks
// of page i while the odd lane finalises page i-1 from the state the even
// lane handed over (a lane shuffle). Both lanes execute the same compression
// instructions on their own data, so a page costs the wave two compressions
// (int64 ids; one for int32) instead of three on one lane.
#include "mkv_device.h"

namespace mkv {
namespace {

__global__ __launch_bounds__(kThreads) void block_hash_kernel(const uint8_t* tokens,
                                                             const int64_t* tok_off,
                                                             const int64_t* page_off,
                                                             int32_t num_requests,
                                                             int32_t token_bytes, uint64_t* out,
                                                             int32_t* err) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t r = t >> 1;
  const bool finisher = (t & 1) != 0;
  // Both lanes of a pair run the same number of steps (the shuffles need the
  // partner active); a pair past the last request runs none.
  int64_t pages = 0, o0 = 0, t0 = 0;
  if (r < num_requests) {
    t0 = tok_off[r];
    const int64_t t1 = tok_off[r + 1];
    o0 = page_off[r];
    const int64_t o1 = page_off[r + 1];
    if (t1 < t0 || o1 - o0 != (t1 - t0) / 16) {
      // the caller's offsets disagree with the token counts
      if (!finisher) raise_err(err, MKV_DEVERR_TABLE);
    } else {
      pages = (t1 - t0) / 16;
    }
  }
  const uint32_t* p = reinterpret_cast<const uint32_t*>(tokens + t0 * token_bytes);
  const int bpp = token_bytes * 16 / 64;  // 64-byte blocks per page: 2 (int64), 1 (int32)
  const uint64_t page_bytes = (uint64_t)token_bytes * 16u;
  Sha256 s;  // even lane: the running state; odd lane: the state it finalises
  sha256_init(s);
  // the even lane loads block b+1 while block b is compressed
  uint32_t next[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) next[j] = 0;
  if (!finisher && pages > 0) {
#pragma unroll
    for (int j = 0; j < 16; ++j) next[j] = p[j];
  }
  int64_t b = 0;  // the even lane's next block
  // Step i: the even lane absorbs page i (if i < pages), the odd lane
  // finalises page i-1 (if i > 0).
  for (int64_t i = 0; i <= pages; ++i) {
    for (int k = 0; k < bpp; ++k) {
      if (k > 0 && i == pages) break;  // nothing left to absorb
      uint32_t w[16];
      if (!finisher) {
#pragma unroll
        for (int j = 0; j < 16; ++j) w[j] = bswap32(next[j]);
        if (b + 1 < pages * bpp) {
          const uint32_t* q = p + 16 * (b + 1);
#pragma unroll
          for (int j = 0; j < 16; ++j) next[j] = q[j];
        }
        ++b;
      } else if (k == 0) {
        sha256_pad_block(w, (uint64_t)i * page_bytes);
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) w[j] = 0;  // idle: the result is replaced below
      }
      sha256_compress(s, w);
      if (finisher && k == 0 && i > 0) out[o0 + i - 1] = ((uint64_t)s.h[0] << 32) | s.h[1];
    }
    // the odd lane takes the state after page i
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t v = __shfl_xor(s.h[j], 1);
      if (finisher) s.h[j] = v;
    }
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
  // two lanes per request
  hipLaunchKernelGGL(block_hash_kernel, dim3((2 * (int64_t)num_requests + kThreads - 1) / kThreads),
                     dim3(kThreads), 0, as_stream(stream), (const uint8_t*)tokens, tok_offsets,
                     page_offsets, num_requests, token_bytes, out, err);
  return check_launch("mkv_block_hash_sha256");
}
