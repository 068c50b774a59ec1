// mkv_hash.hip — per-page SHA-256 prefix hashes for the prefix cache (gfx950).
//
// The key of a prefix is the first 8 bytes of SHA-256 over its token ids as
// little-endian integers (muserve/model/prefix_cache.py:31-34). A page is 16
// tokens, i.e. 128 bytes of int64 ids = exactly two SHA-256 blocks (one for
// int32 ids), so the hash of "the prefix ending at page i" is the running
// SHA-256 state after page i, finalised with one constant-length padding
// block. A request's pages form a dependent chain of compressions, and the
// kernel is bound by instruction issue along that chain, not by HBM.
//
// Two adjacent lanes share a request: the even lane absorbs the token blocks
// of page i while the odd lane finalises page i-1 from the state the even
// lane handed over (a lane shuffle), so a page costs the chain two
// compressions (int64 ids; one for int32) instead of three.
//
// A workgroup is two waves over the same 64 lanes (32 requests). The message
// schedule of a block does not depend on the running state, so the second
// wave computes K[t] + W[t] for every block one step ahead into LDS, and the
// first wave runs only the 64 rounds of each compression: about 880
// instructions per compression on the chain instead of about 1,550.
#include "mkv_device.h"

namespace mkv {
namespace {

constexpr int kHashPairs = 32;    // requests per workgroup (two lanes each)
constexpr int kHashThreads = 128;  // wave 0: rounds; wave 1: message schedules

// K[t] + W[t], t < 64, of one block (16 big-endian words), as 16 quads down
// the lane's column of an LDS buffer laid out [quad][lane].
__device__ __forceinline__ void sha256_kw_store(const uint32_t blk[16], uint4* col) {
  uint32_t w[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) w[i] = blk[i];
  uint32_t q[4];
#pragma unroll
  for (int t = 0; t < 64; ++t) {
    uint32_t wt;
    if (t < 16) {
      wt = w[t];
    } else {
      const uint32_t w15 = w[(t - 15) & 15], w2 = w[(t - 2) & 15];
      const uint32_t s0 = xor3(rotr32(w15, 7), rotr32(w15, 18), w15 >> 3);
      const uint32_t s1 = xor3(rotr32(w2, 17), rotr32(w2, 19), w2 >> 10);
      wt = w[t & 15] = w[t & 15] + s0 + w[(t - 7) & 15] + s1;
    }
    q[t & 3] = wt + kSha256K[t];
    if ((t & 3) == 3) col[(t >> 2) * 64] = uint4{q[0], q[1], q[2], q[3]};
  }
}

// One compression whose K[t] + W[t] come from the lane's LDS column.
__device__ __forceinline__ void sha256_rounds_kw(Sha256& s, const uint4* col) {
  uint32_t kw[64];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint4 v = col[i * 64];
    kw[4 * i] = v.x;
    kw[4 * i + 1] = v.y;
    kw[4 * i + 2] = v.z;
    kw[4 * i + 3] = v.w;
  }
  uint32_t a = s.h[0], b = s.h[1], c = s.h[2], d = s.h[3];
  uint32_t e = s.h[4], f = s.h[5], g = s.h[6], h = s.h[7];
#pragma unroll
  for (int t = 0; t < 64; ++t) {
    const uint32_t S1 = xor3(rotr32(e, 6), rotr32(e, 11), rotr32(e, 25));
    const uint32_t ch = (e & f) ^ (~e & g);
    const uint32_t t1 = h + S1 + ch + kw[t];
    const uint32_t S0 = xor3(rotr32(a, 2), rotr32(a, 13), rotr32(a, 22));
    // majority: one v_bitop3_b32 (truth table 0xe8, symmetric in its inputs)
    const uint32_t maj = __builtin_amdgcn_bitop3_b32(a, b, c, 0xe8);
    h = g; g = f; f = e; e = d + t1;
    d = c; c = b; b = a; a = t1 + S0 + maj;
  }
  s.h[0] += a; s.h[1] += b; s.h[2] += c; s.h[3] += d;
  s.h[4] += e; s.h[5] += f; s.h[6] += g; s.h[7] += h;
}

__global__ __launch_bounds__(kHashThreads) void block_hash_kernel(const uint8_t* tokens,
                                                                 const int64_t* tok_off,
                                                                 const int64_t* page_off,
                                                                 int32_t num_requests,
                                                                 int32_t token_bytes,
                                                                 uint64_t* out, int32_t* err) {
  __shared__ uint4 kw[2][16][64];  // K+W of the blocks of two consecutive steps
  const int lane = threadIdx.x & 63;
  const bool rounds = threadIdx.x < 64;  // else: the schedule wave
  const int64_t r = (int64_t)blockIdx.x * kHashPairs + (lane >> 1);
  const bool finisher = (lane & 1) != 0;
  int64_t pages = 0, o0 = 0, t0 = 0;
  if (r < num_requests) {
    t0 = tok_off[r];
    const int64_t t1 = tok_off[r + 1];
    o0 = page_off[r];
    const int64_t o1 = page_off[r + 1];
    if (t1 < t0 || o1 - o0 != (t1 - t0) / 16) {
      // the caller's offsets disagree with the token counts
      if (rounds && !finisher) raise_err(err, MKV_DEVERR_TABLE);
    } else {
      pages = (t1 - t0) / 16;
    }
  }
  const int bpp = token_bytes * 16 / 64;  // 64-byte blocks per page: 2 (int64), 1 (int32)
  const uint64_t page_bytes = (uint64_t)token_bytes * 16u;
  const int64_t nblk = pages * bpp;
  // Step s < nblk + 1: the even lane absorbs block s (s < nblk); the odd lane
  // finalises page s / bpp - 1 at the first block of page s / bpp (1 <= s /
  // bpp <= pages). Both waves run the workgroup's largest step count.
  int64_t steps = pages > 0 ? nblk + 1 : 0;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const int64_t o = __shfl_xor(steps, off);
    steps = o > steps ? o : steps;
  }
  const uint32_t* p = reinterpret_cast<const uint32_t*>(tokens + t0 * token_bytes);
  uint4* col_base = &kw[0][0][lane];

  Sha256 st;  // rounds wave: the even lane's running state; the odd lane's to finalise
  sha256_init(st);
  // schedule wave: the even lane holds the next block's words
  uint32_t next[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) next[j] = 0;
  if (!rounds && !finisher && nblk > 0) {
#pragma unroll
    for (int j = 0; j < 16; ++j) next[j] = p[j];
  }
  // Iteration s: the rounds wave compresses step s (from buffer s & 1) while
  // the schedule wave fills step s + 1 (buffer (s + 1) & 1); one barrier
  // ends the iteration, so both waves run steps + 1 of them. Step u is block
  // k of page i (u = i * bpp + k), kept as counters: the rounds wave's for s,
  // the schedule wave's for s + 1.
  int64_t i = 0;
  int k = rounds ? -1 : 0;  // the rounds wave's first iteration has no step
  for (int64_t s = -1; s < steps; ++s) {
    if (rounds) {
      if (s >= 0) {
        sha256_rounds_kw(st, col_base + (s & 1) * 16 * 64);
        if (finisher && k == 0 && i >= 1 && i <= pages)
          out[o0 + i - 1] = ((uint64_t)st.h[0] << 32) | st.h[1];
        if (k == bpp - 1) {  // end of page i: the odd lane takes the state
          // adjacent lanes swap through DPP quad_perm [1,0,3,2] (lane ^ 1),
          // a VALU operand modifier rather than an LDS permute round trip
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const uint32_t v = (uint32_t)__builtin_amdgcn_mov_dpp((int)st.h[j], 0xb1, 0xf, 0xf, false);
            if (finisher) st.h[j] = v;
          }
        }
      }
    } else {
      const int64_t u = s + 1;  // the step to schedule: block k of page i
      uint32_t w[16];
      bool any = false;
      if (!finisher) {
        if (u < nblk) {
#pragma unroll
          for (int j = 0; j < 16; ++j) w[j] = bswap32(next[j]);
          if (u + 1 < nblk) {
            const uint32_t* q = p + 16 * (u + 1);
#pragma unroll
            for (int j = 0; j < 16; ++j) next[j] = q[j];
          }
          any = true;
        }
      } else {
        if (k == 0 && i >= 1 && i <= pages) {
          sha256_pad_block(w, (uint64_t)i * page_bytes);
          any = true;
        }
      }
      if (any) sha256_kw_store(w, col_base + (u & 1) * 16 * 64);
    }
    if (++k == bpp) {
      k = 0;
      ++i;
    }
    __syncthreads();
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
  // two lanes per request, kHashPairs requests per workgroup
  hipLaunchKernelGGL(block_hash_kernel,
                     dim3(((int64_t)num_requests + kHashPairs - 1) / kHashPairs),
                     dim3(kHashThreads), 0, as_stream(stream), (const uint8_t*)tokens,
                     tok_offsets, page_offsets, num_requests, token_bytes, out, err);
  return check_launch("mkv_block_hash_sha256");
}
