// mkv_hash.hip — per-page SHA-256 prefix hashes for the prefix cache (gfx950).
//
// The key of a prefix is the first 8 bytes of SHA-256 over its token ids as
// little-endian integers (muserve/model/prefix_cache.py:31-34). A page is 16
// tokens, i.e. 128 bytes of int64 ids = exactly two SHA-256 blocks, so the
// hash of "the prefix ending at page i" is the running SHA-256 state after
// page i, finalised with one constant padding block. A request's pages form a
// dependent chain; requests are independent, so one lane walks one request
// and a launch covers a whole batch of requests. The work is integer ALU and
// latency bound, not HBM bound: per page two chained compressions, plus a
// finalisation that runs interleaved with the next page's first compression,
// while the next block's words are already being loaded.
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
  const int64_t bpp = token_bytes * 16 / 64;  // 64-byte blocks per page: 2 (int64), 1 (int32)
  const int64_t nblocks = pages * bpp;
  const uint64_t page_bytes = (uint64_t)token_bytes * 16u;
  Sha256 s;
  sha256_init(s);
  // Block b+1's words are loaded while block b is compressed; a page's
  // finalisation (one more compression of a copy of the state) runs
  // interleaved with the next block's compression.
  uint32_t next[16];
  if (nblocks > 0) {
#pragma unroll
    for (int j = 0; j < 16; ++j) next[j] = p[j];
  }
  Sha256 fin;
  uint32_t pad[16];
  bool pending = false;  // fin holds a page state awaiting its padding block
  int64_t pending_page = 0;
  for (int64_t b = 0; b < nblocks; ++b) {
    uint32_t w[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) w[j] = bswap32(next[j]);
    if (b + 1 < nblocks) {
      const uint32_t* q = p + 16 * (b + 1);
#pragma unroll
      for (int j = 0; j < 16; ++j) next[j] = q[j];
    }
    if (pending) {
      sha256_compress2(s, w, fin, pad);
      out[o0 + pending_page] = ((uint64_t)fin.h[0] << 32) | fin.h[1];
      pending = false;
    } else {
      sha256_compress(s, w);
    }
    if (bpp == 1 || (b & 1)) {  // block b ends a page
      pending_page = bpp == 1 ? b : b >> 1;
      fin = s;
      sha256_pad_block(pad, (uint64_t)(pending_page + 1) * page_bytes);
      pending = true;
    }
  }
  if (pending)
    out[o0 + pending_page] =
        sha256_final_aligned_u64(fin, (uint64_t)(pending_page + 1) * page_bytes);
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
