// mkv_attn.hip — paged decode attention reading the KV pool directly (gfx950).
//
// One decode query token per sequence attends to the first seq_lens[b] cached
// tokens of its block table: for each of the G query heads sharing a KV head,
// softmax(q k^T * scale) v over the sequence, computed in fp32, written in
// the pool's 16-bit type. This is the interface of the paged decode kernel the
// reference wraps (muserve/kernels/attention.py:29-42) and the math of its
// contiguous decode path (muserve/model/qwen35_layer_v2.py:493-502), without
// the padded gather.
//
// Each cached K/V byte is read once and carries G flop, so the bound is HBM.
// What decides the rate is how many page reads are in flight and how they are
// issued (on MI355X random 8 KiB page reads stream at 6.8 TB/s only with the
// non-temporal bit set; without it ~6.0 TB/s whatever the depth):
//   * Work split: the (sequence, KV head) pairs' pages form one flat list
//     (pair-major, pages in table order). Every wave of the grid (the
//     resident workgroups, 4 waves each) takes an equal contiguous span of
//     it. No counters, no atomics, no tail of short items: spans differ by
//     at most one page. Each workgroup computes the pairs' page prefix in LDS
//     in its prologue; workgroup 0 also leaves it in the workspace.
//   * Shared pages (ids below shared_pages, handed to many sequences by
//     prefix reuse) are read through the caches, every other page streams
//     past them. With shared pages the spans are aligned to the pairs: each
//     pair's page count is rounded up to a multiple of the span, so every
//     pair reads its page i at the same point of a wave's span, and the
//     pairs sharing a page read it at once while L2 still holds it. The
//     pairs are taken in the order of their first page id (a bitonic sort in
//     each workgroup's prologue), and the spans go to the XCDs in contiguous
//     ranges, so the pairs sharing a prefix share one XCD's L2 (prefix
//     serving workload: L2 hit rate 0.12 with equal spans, 0.37 aligned,
//     0.63 sorted; 181 -> 135 -> 132 us per layer serial, 200 -> 160 -> 147
//     us beside the prefill attention).
//   * Loads: a wave streams its span's K and V planes page by page straight
//     into its own LDS slots with global_load_lds_dwordx4 (16 bytes a lane,
//     1 KiB per instruction, non-temporal). The next page's K is issued as
//     soon as this page's scores have read the K slot, its V as soon as P V
//     has read the V slot, so up to a page is in flight per wave while the
//     wave computes. Completion is tracked with exact vmcnt waits. A pair's
//     query rows ride the same stream, ahead of its first K plane. Page ids
//     come from the table through scalar loads, which do not touch vmcnt.
//   * LDS layout: chunk c of a cached row r is stored at chunk c ^ (r & 15)
//     of that row (the DMA lanes fetch the permuted chunks), so the MFMA
//     operand reads of 16 rows x 16 bytes hit 16 distinct bank groups.
//   * Scores on MFMA (v_mfma_f32_16x16x32_{bf16,f16}; fp8 codes converted
//     exactly to bf16): A = the 16 K rows of the page from LDS, B = the G
//     query heads (zero columns above G) held in registers for the pair.
//     Online softmax per head in fp32 (exp2 with log2 e folded into the
//     scale); the page's probabilities go through a wave-private LDS tile.
//   * P V on the VALU: a lane owns 8 dims of every head over 8 of the 16
//     tokens (half waves take the two halves of the page); a V row is one
//     16-byte LDS read per lane. The halves are summed at the segment's end.
//   * A pair wholly inside one span is finished by its wave (normalised
//     output). A pair cut by span boundaries leaves (max, sum, unnormalised
//     output) per piece in the workspace, at most two per wave; a second
//     kernel merges them and also writes the zeros of empty pairs.
#include <math.h>

#include <mutex>
#include <type_traits>

#include "mkv_device.h"

namespace mkv {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kHeadDim = 256;
constexpr int kRowBytes = kHeadDim * 2;  // one 16-bit K or V row of one KV head
constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr int kPageTokens = 16;
constexpr int kMaxPairs = 4096;  // batch x KV heads whose page prefix fits in LDS
constexpr int kSortPairs = 1024;  // pairs sorted by first page for aligned spans
constexpr int kXcds = 8;          // MI355X: workgroups go round robin over 8 XCDs
constexpr int64_t kHeaderBytes = 256;
constexpr size_t kLdsPerCu = 160 * 1024;  // MI355X

struct AttnArgs {
  const uint8_t* q;  // [B, Hkv * G, 256] 16-bit
  const uint8_t* k;  // [P, 16, Hkv, 256] 16-bit or e4m3fn codes; contiguous mode [B, S, Hkv, 256]
  const uint8_t* v;
  const float* ks;   // fp8 caches: [P, 16, Hkv] fp32 scales of K and V
  const float* vs;
  const int32_t* table;  // [B, tstride] int32 (paged mode)
  const int32_t* lens;   // [B] int32
  uint8_t* out;          // [B, Hkv * G, 256] 16-bit
  int64_t* hdr;          // workspace header: [0] span S (pages per wave), [1] total pages T
  int32_t* pre;          // [pairs + 1]: each pair's first flat page (the prefix of the page
                         //  counts; aligned spans: the virtual start, in the sorted order)
  int32_t* pend;         // [pairs]: each pair's flat page end (its start + its page count)
  float* part;           // [waves, 2, G, 256] unnormalised outputs of cut pairs' pieces
  float* ml;             // [waves, 2, G, 2] their (max, sum), log2 units
  int64_t num_pages, tstride;
  int64_t shared_below;  // page ids below it are loaded through the caches
  int64_t seq_rows;      // contiguous mode: rows per sequence (0: paged)
  int32_t twidth, hkv, max_len, pairs;
  float scale_log2;      // softmax_scale * log2(e)
  int32_t* err;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return bits_f32(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return bits_f32(w & 0xffff0000u); }
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float f16_lo(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
__device__ __forceinline__ float f16_hi(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// One 16 x 16 x 32 MFMA step of the scores over 16-bit rows: fp16 pools use
// the fp16 instruction, bf16 pools (and fp8 codes converted to bf16) the
// bf16 one. Operands travel as raw 16-byte registers.
template <bool F16>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// An output element in the pool's 16-bit type: round to nearest even (fp16
// overflows to infinity, as torch's float -> half conversion does).
template <bool F16>
__device__ __forceinline__ uint16_t out_bits(float x) {
  if constexpr (F16)
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  else
    return f32_to_bf16_rne(x);
}

// Orders this wave's LDS writes before its later LDS reads (other lanes').
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Eight e4m3fn codes (little-endian bytes of lo, hi) as eight bf16: exact,
// every e4m3fn value is a bf16 value. gfx950 converts a code pair straight to
// a bf16 pair (v_cvt_scalef32_pk_bf16_fp8, scale 1; mkv_check_conversions
// checks it on every code).
__device__ __forceinline__ u32x4 fp8x8_bf16(uint32_t lo, uint32_t hi) {
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)lo, 1.0f, false);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)lo, 1.0f, true);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)hi, 1.0f, false);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)hi, 1.0f, true);
  return u32x4{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
               __builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, d)};
}

// ---- direct-to-LDS loads and their completion ---------------------------------
//
// The loads are issued from inline assembly, so the compiler neither inserts
// waits for them nor reorders LDS accesses across them ("memory" clobber);
// every wait on them is explicit below. M0 holds the LDS destination of the
// lane-0 bytes (the hardware adds 16 or 4 bytes per lane); the compiler keeps
// nothing in M0 across these statements in this file (no LDS DMA builtins,
// GWS, message or movrel instructions). Before a slot is refilled, the wave's
// earlier LDS reads of it must have returned: lgkmcnt(0) first.

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// A wave-uniform pointer in scalar registers (the compiler cannot always
// prove uniformity through the index arithmetic).
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t u = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
}
// 16 bytes per lane from base + voff (saddr form: base scalar, voff per lane)
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(uniform_ptr(base))
               : "memory");
}
// the same through the caches (pages several sequences read: a prefix
// shared through the block manager)
__device__ __forceinline__ void dma16_cached(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(uniform_ptr(base))
               : "memory");
}
// 4 bytes per lane from a per-lane 64-bit address
__device__ __forceinline__ void dma4(const void* addr, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off nt"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(addr)
               : "memory");
}
__device__ __forceinline__ void lds_reads_done() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
template <int N>
__device__ __forceinline__ void vm_wait_n() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Waits until at most n vector-memory operations of this wave are
// outstanding (n wave-uniform). The loads return in issue order, so the
// loads issued before the youngest n are then complete.
__device__ __forceinline__ void vm_wait(int n) {
  switch (n) {
#define MKV_VMW(k) \
  case k: vm_wait_n<k>(); break;
    MKV_VMW(0) MKV_VMW(1) MKV_VMW(2) MKV_VMW(3) MKV_VMW(4) MKV_VMW(5) MKV_VMW(6) MKV_VMW(7)
    MKV_VMW(8) MKV_VMW(9) MKV_VMW(10) MKV_VMW(11) MKV_VMW(12) MKV_VMW(13) MKV_VMW(14) MKV_VMW(15)
    MKV_VMW(16) MKV_VMW(17) MKV_VMW(18) MKV_VMW(19) MKV_VMW(20) MKV_VMW(21) MKV_VMW(22) MKV_VMW(23)
    MKV_VMW(24) MKV_VMW(25) MKV_VMW(26) MKV_VMW(27) MKV_VMW(28) MKV_VMW(29) MKV_VMW(30) MKV_VMW(31)
    MKV_VMW(32) MKV_VMW(33) MKV_VMW(34) MKV_VMW(35) MKV_VMW(36) MKV_VMW(37) MKV_VMW(38) MKV_VMW(39)
    MKV_VMW(40) MKV_VMW(41) MKV_VMW(42) MKV_VMW(43) MKV_VMW(44) MKV_VMW(45) MKV_VMW(46) MKV_VMW(47)
    MKV_VMW(48) MKV_VMW(49) MKV_VMW(50) MKV_VMW(51) MKV_VMW(52) MKV_VMW(53) MKV_VMW(54) MKV_VMW(55)
    MKV_VMW(56) MKV_VMW(57) MKV_VMW(58) MKV_VMW(59) MKV_VMW(60) MKV_VMW(61) MKV_VMW(62) MKV_VMW(63)
#undef MKV_VMW
    default: vm_wait_n<0>(); break;  // never taken: a wave has at most 63 loads outstanding
  }
}

// Geometry of one pool kind (bf16 / fp16 / fp8) and query-group size G.
// A wave's loads go through a ring of kRing unit slots: unit 2i is page i's K
// plane (with the pair's query rows ahead of it when the page starts a pair,
// and for fp8 the page's K and V scales), unit 2i+1 its V plane. Unit u+kRing
// is issued as soon as unit u has been read, so kRing-1 units are in flight
// while the wave computes on one.
template <int G, bool FP8>
struct Geo {
  static constexpr int kCodeRow = FP8 ? kHeadDim : kRowBytes;  // bytes of a cached row
  static constexpr int kPlane = kPageTokens * kCodeRow;        // a page's K (or V) bytes
  static constexpr int kChunks = kCodeRow / 16;                // 16-byte chunks per row
  static constexpr int kPlaneIns = kPlane / 1024;              // instructions per plane
  static constexpr int kRing = 2;                              // unit slots per wave
  // query-row slots: with two slots a pair's rows are issued after the pair
  // two pairs back has read its own (at least four units earlier)
  static constexpr int kQSlots = kRing == 2 ? 1 : 2;
  static constexpr int kQBytes = G * kRowBytes < 1024 ? 1024 : G * kRowBytes;
  static constexpr int kQIns = kQBytes / 1024;
  static constexpr int kScaleBytes = FP8 ? 256 : 0;  // K scales, V scales (64 B each) + copies
  static constexpr int kScaleIns = FP8 ? 1 : 0;
  // per-wave LDS: unit slots, scale slots, query rows, probability tile
  static constexpr int kOffU = 0;
  static constexpr int kOffS = kOffU + kRing * kPlane;
  static constexpr int kOffQ = kOffS + kRing * kScaleBytes;
  static constexpr int kOffP = kOffQ + kQSlots * kQBytes;
  static constexpr int kWaveBytes = kOffP + kPageTokens * G * 4;
  static_assert(kWaveBytes % 16 == 0, "16-byte aligned slots");
  static_assert(kPlaneIns + kScaleIns + kQIns <= 15, "a unit's loads fit a 4-bit count");
  static_assert(kRing >= 2 && kRing <= 4, "ring of 2 to 4 units");
};

// Dynamic LDS of one workgroup: the pairs' page prefix and lengths, then the
// four waves' slots.
template <int G, bool FP8>
inline size_t attn_lds_bytes(int32_t pairs) {
  const size_t meta = ((size_t)(pairs + 1) * 8 + 15) / 16 * 16;
  return meta + (size_t)kAttnWaves * Geo<G, FP8>::kWaveBytes;
}

// SHARED: some pages (ids below shared_below) are read through the caches;
// without it every page streams (the launch picks the variant, so a batch
// with no shared pages carries no code or registers for them).
template <int G, bool FP8, bool F16, bool SHARED>
__global__ __launch_bounds__(kAttnThreads, G == 8 ? 1 : 2) void attn_span_kernel(AttnArgs a) {
  static_assert(G >= 1 && G <= 8, "query heads per KV head");
  using Gm = Geo<G, FP8>;
  constexpr int R = Gm::kRing;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ int32_t wave_tot[kAttnWaves];
  int32_t* pre_l = reinterpret_cast<int32_t*>(lds);  // [pairs + 1]
  int32_t* len_l = pre_l + (a.pairs + 1);             // [pairs]
  const size_t meta = ((size_t)(a.pairs + 1) * 8 + 15) / 16 * 16;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // ---- prologue: lengths (clamped to the table and the launch's bound) and
  // the exclusive prefix of the pairs' page counts, 256 pairs per round
  const int64_t cap = (int64_t)a.twidth * kPageTokens < a.max_len
                          ? (int64_t)a.twidth * kPageTokens
                          : (int64_t)a.max_len;
  int32_t total = 0;
  for (int base = 0; base < a.pairs; base += kAttnThreads) {
    const int pr = base + tid;
    int32_t cnt = 0;
    if (pr < a.pairs) {
      int64_t len = ld_const(a.lens + pr / a.hkv);
      if (len > cap || len < 0) {
        if (blockIdx.x == 0 && pr % a.hkv == 0) raise_err(a.err, MKV_DEVERR_TABLE);
        len = len < 0 ? 0 : cap;
      }
      len_l[pr] = (int32_t)len;
      cnt = (int32_t)((len + kPageTokens - 1) / kPageTokens);
    }
    int32_t incl = cnt;
#pragma unroll
    for (int dd = 1; dd < 64; dd <<= 1) {
      const int32_t o = __shfl_up(incl, dd);
      if (lane >= dd) incl += o;
    }
    if (lane == 63) wave_tot[wave] = incl;
    __syncthreads();
    int32_t at = total + incl - cnt, round = 0;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      at += w < wave ? wave_tot[w] : 0;
      round += wave_tot[w];
    }
    if (pr < a.pairs) pre_l[pr] = at;
    total += round;
    __syncthreads();  // wave_tot is rewritten by the next round
  }
  if (tid == 0) pre_l[a.pairs] = total;
  __syncthreads();
  int64_t T = total;
  const int64_t W = (int64_t)gridDim.x * kAttnWaves;
  int64_t S = (T + W - 1) / W;
  // With shared pages, every pair's pages start a span: the prefix is over
  // the pairs' page counts rounded up to a multiple of the span (a virtual
  // prefix; a wave's span then lies inside one pair), and the span is the
  // least that still fits the waves. Every pair reads its page i at the same
  // point of its waves' spans, so a page that prefix reuse gives many pairs is
  // read by all of them at once, while the first read still holds it in L2.
  // Equal spans over the pairs as they come (the other case) stagger those
  // reads over the whole launch. Used when at most half the waves are pairs.
  bool aligned = false, sorted = false;
  // Sorted (aligned, paged, at most kSortPairs pairs): the virtual prefix
  // takes the pairs in the order of their sequence's first page id, so pairs
  // sharing a prefix get adjacent spans; keys and the ranks' starts live in
  // the wave slots' LDS until the loads start.
  uint64_t* key = reinterpret_cast<uint64_t*>(lds + meta);          // [kSortPairs]
  int32_t* vps = reinterpret_cast<int32_t*>(key + kSortPairs);      // [pairs + 1] by rank
  if constexpr (SHARED) {
    auto block_sum = [&](int64_t v) __attribute__((always_inline)) {
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
      __syncthreads();  // wave_tot's earlier readers are done
      if (lane == 0) wave_tot[wave] = (int32_t)v;
      __syncthreads();
      int64_t t = 0;
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) t += wave_tot[w];
      return t;
    };
    auto pages_of = [&](int p) __attribute__((always_inline)) {
      return (int64_t)((len_l[p] + kPageTokens - 1) / kPageTokens);
    };
    int64_t mine = 0;
    for (int p = tid; p < a.pairs; p += kAttnThreads) mine += pages_of(p) > 0 ? 1 : 0;
    const int64_t np = block_sum(mine);
    if (np > 0 && 2 * np <= W && 2 * T + W < (int64_t)INT_MAX) {
      // the least span in [S, ceil(T / (W - np))] whose rounded counts fit W
      // waves (the upper end always does: each pair rounds up by under one)
      int64_t lo = S, hi = (T + (W - np) - 1) / (W - np);
      while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        int64_t need = 0;
        for (int p = tid; p < a.pairs; p += kAttnThreads) need += (pages_of(p) + mid - 1) / mid;
        if (block_sum(need) <= W) hi = mid; else lo = mid + 1;
      }
      S = lo;
      aligned = true;
      sorted = a.seq_rows == 0 && a.pairs <= kSortPairs;
      __syncthreads();  // the last block_sum's readers are done with wave_tot
      if (sorted) {  // bitonic sort of (first page id, pair) in LDS; keys are unique
        int n2 = 2;
        while (n2 < a.pairs) n2 <<= 1;
        for (int i = tid; i < n2; i += kAttnThreads) {
          uint64_t kk = ~0ull;  // padding sorts last
          if (i < a.pairs) {
            const uint32_t first =
                pages_of(i) > 0 ? (uint32_t)ld_const(a.table + (int64_t)(i / a.hkv) * a.tstride)
                                : 0xffffffffu;  // an empty pair: after every page id
            kk = (uint64_t)first << 32 | (uint32_t)i;
          }
          key[i] = kk;
        }
        __syncthreads();
        for (int k = 2; k <= n2; k <<= 1) {
          for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < n2; i += kAttnThreads) {
              const int x = i ^ j;
              if (x > i) {
                const uint64_t u = key[i], v = key[x];
                if ((u > v) == ((i & k) == 0)) {
                  key[i] = v;
                  key[x] = u;
                }
              }
            }
            __syncthreads();
          }
        }
      }
      int32_t vt = 0;
      for (int base = 0; base < a.pairs; base += kAttnThreads) {
        const int rk = base + tid;  // rank: position in the sorted order (or the pairs' own)
        const int pr = rk < a.pairs ? (sorted ? (int)(uint32_t)key[rk] : rk) : 0;
        const int32_t cnt =
            rk < a.pairs ? (int32_t)((pages_of(pr) + S - 1) / S * S) : 0;
        int32_t incl = cnt;
#pragma unroll
        for (int dd = 1; dd < 64; dd <<= 1) {
          const int32_t o = __shfl_up(incl, dd);
          if (lane >= dd) incl += o;
        }
        if (lane == 63) wave_tot[wave] = incl;
        __syncthreads();
        int32_t at = vt + incl - cnt, round = 0;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) {
          at += w < wave ? wave_tot[w] : 0;
          round += wave_tot[w];
        }
        if (rk < a.pairs) {
          pre_l[pr] = at;
          vps[rk] = at;
        }
        vt += round;
        __syncthreads();  // wave_tot is rewritten by the next round
      }
      if (tid == 0) {
        pre_l[a.pairs] = vt;
        vps[a.pairs] = vt;
      }
      __syncthreads();
      T = vt;
    }
  }
  // The pair holding flat page f: the last pair p with pre[p] <= f (empty
  // pairs share their successor's prefix, so it is never empty). Not used
  // once sorted: a wave's span then lies in the one pair found below.
  auto pair_of = [&](int64_t f) __attribute__((always_inline)) {
    int lo = 0, hi = a.pairs - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (pre_l[mid] <= f) lo = mid; else hi = mid - 1;
    }
    return __builtin_amdgcn_readfirstlane(lo);
  };
  // The flat end of pair p's pages (the next pair's start, unless aligned).
  auto pair_end = [&](int p) __attribute__((always_inline)) {
    if constexpr (SHARED)
      return (int64_t)pre_l[p] + (len_l[p] + kPageTokens - 1) / kPageTokens;
    else
      return (int64_t)pre_l[p + 1];
  };
  if (blockIdx.x == 0) {  // for the merge kernel
    for (int p = tid; p <= a.pairs; p += kAttnThreads) a.pre[p] = pre_l[p];
    for (int p = tid; p < a.pairs; p += kAttnThreads) a.pend[p] = (int32_t)pair_end(p);
    if (tid == 0) {
      a.hdr[0] = S;
      a.hdr[1] = T;
    }
  }
  // Aligned spans go to the XCDs in contiguous ranges: the dispatcher hands
  // workgroup w to XCD w % 8, so workgroup w takes logical block
  // (w % 8) * (grid / 8) + w / 8, and the pairs sharing a prefix (adjacent
  // once sorted) read it through one L2.
  int64_t lb = blockIdx.x;
  if (aligned && gridDim.x % kXcds == 0)
    lb = (int64_t)(blockIdx.x % kXcds) * (gridDim.x / kXcds) + blockIdx.x / kXcds;
  const int64_t gw = lb * kAttnWaves + wave;
  const int64_t s0 = gw * S < T ? gw * S : T;
  int64_t s1 = s0 + S < T ? s0 + S : T;
  int32_t wpair = -1;  // aligned: the one pair of the span
  if (aligned && s0 < s1) {
    if (sorted) {  // the last rank whose virtual start is at or before s0
      int lo = 0, hi = a.pairs - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (vps[mid] <= s0) lo = mid; else hi = mid - 1;
      }
      wpair = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)key[lo]);
    } else {
      wpair = pair_of(s0);
    }
    const int64_t e = pair_end(wpair);  // the span ends with its pair's pages
    s1 = s1 < e ? s1 : e;
  }
  if (sorted) __syncthreads();  // every wave has read the keys before the slots fill
  if (s0 >= s1) return;  // no barrier follows: an idle wave may leave
  // The two resident workgroups of a CU put one wave each on every SIMD, and
  // the SIMD's arbiter favours the older wave: with equal spans the first
  // workgroup's waves finished in ~180 us and the second's in ~220 us (batch
  // 256 decode shape). The two waves take turns at the higher issue priority,
  // page by page, by the parity of their hardware wave slot (HW_ID WAVE_ID).
  const uint32_t wslot = __builtin_amdgcn_s_getreg((3 << 11) | 4) & 1u;

  uint8_t* wl = lds + meta + (size_t)wave * Gm::kWaveBytes;
  float* ptile = reinterpret_cast<float*>(wl + Gm::kOffP);  // [16 tokens][G]
  const uint32_t unit_a = lds_addr(wl + Gm::kOffU);         // slot i at unit_a + i * kPlane
  const uint32_t scale_a = lds_addr(wl + Gm::kOffS);        // slot i at scale_a + i * 256
  const uint32_t q_a = lds_addr(wl + Gm::kOffQ);            // slot i at q_a + i * kQBytes

  // ---- lane constants of the DMA addressing and the LDS reads (relative to
  // a slot's start)
  const int64_t row_stride = (int64_t)a.hkv * Gm::kCodeRow;  // bytes between token rows
  uint32_t voff[Gm::kPlaneIns];  // lane's byte offset in a page plane, per instruction
#pragma unroll
  for (int j = 0; j < Gm::kPlaneIns; ++j) {
    const int p = 64 * j + lane;  // 16-byte position in the slot
    const int r = p / Gm::kChunks;
    const int c = (p % Gm::kChunks) ^ (r & 15);
    voff[j] = (uint32_t)(r * row_stride + c * 16);
  }
  // fp8: lane t < 16 fetches token t's K scale, 16 <= lane < 32 the V scale
  // (lanes 32-63 repeat them into the slot's unused half)
  const int st = lane & 15;
  const float* sbase = ((lane >> 4) & 1) ? a.vs : a.ks;
  const int n = lane & 15, g = lane >> 4;     // MFMA lane roles: row / head n, group g
  const int hf = lane >> 5, c8 = lane & 31;   // P V roles: token half, 8-dim chunk
  uint32_t koff[FP8 ? 4 : 8];                 // K operand reads
  if constexpr (FP8) {
#pragma unroll
    for (int r = 0; r < 4; ++r) koff[r] = (n * 16 + ((4 * r + g) ^ n)) * 16;
  } else {
#pragma unroll
    for (int s = 0; s < 8; ++s) koff[s] = (n * 32 + ((4 * s + g) ^ n)) * 16;
  }
  uint32_t voffr[8];  // V row reads: token 8 hf + k, chunk c8
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int t = 8 * hf + k;
    if constexpr (FP8)
      voffr[k] = (t * 16 + ((c8 >> 1) ^ t)) * 16 + (c8 & 1) * 8;
    else
      voffr[k] = (t * 32 + (c8 ^ t)) * 16;
  }
  auto lds_ld16 = [](uint32_t addr) __attribute__((always_inline)) {
    return *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(addr);
  };
  auto lds_ld8 = [](uint32_t addr) __attribute__((always_inline)) {
    return *reinterpret_cast<const __attribute__((address_space(3))) u32x2*>(addr);
  };

  // ---- the issue side walks the span's units in order. Every lambda here
  // is forced inline: a by-reference closure left out of line keeps the
  // locals it captures (and a copy of the arguments) in scratch memory, and
  // a scratch load waits for every outstanding page load (the 16-bit
  // kernels ran 6x slower that way). Indices stay 32-bit where they can: a
  // 64-bit modulo by the head count is a long software sequence per page.
  const int64_t nunits = 2 * (s1 - s0);
  int64_t iu = 0;                    // next unit to issue
  int32_t ip = wpair >= 0 ? wpair : pair_of(s0);  // pair of the page being issued
  int64_t ipre0 = pre_l[ip], ipre1 = pair_end(ip);
  int64_t irow = 0;                  // first cached row of that page
  int64_t irows = kPageTokens;       // its rows inside a contiguous sequence's storage
  bool icached = false;              // its planes through the caches (a shared page)
  uint32_t iqn = 0;                  // pairs whose query rows were issued
  uint32_t badbits = 0;              // bit (f - s0) & 31: page id outside the pool
  // unit sizes in flight (4 bits each, oldest lowest) and their sum
  uint32_t fifo = 0;
  int fifo_n = 0, fifo_total = 0;
  // one page plane into a slot; rows of a contiguous sequence's last page
  // past its end are not read (the lane's row is clamped to the last valid
  // one, only on that page)
  auto issue_plane = [&](const uint8_t* base, uint32_t slot_a) __attribute__((always_inline)) {
    if (SHARED && icached) {  // uniform branches: one per plane
#pragma unroll
      for (int jj = 0; jj < Gm::kPlaneIns; ++jj) dma16_cached(base, voff[jj], slot_a + jj * 1024);
    } else if (irows >= kPageTokens) {
#pragma unroll
      for (int jj = 0; jj < Gm::kPlaneIns; ++jj) dma16(base, voff[jj], slot_a + jj * 1024);
    } else {  // only a contiguous sequence's last page
#pragma unroll
      for (int jj = 0; jj < Gm::kPlaneIns; ++jj) {
        const int p = 64 * jj + lane;
        int r = p / Gm::kChunks;
        const int c = (p % Gm::kChunks) ^ (r & 15);
        if (r >= irows) r = (int)irows - 1;
        dma16(base, (uint32_t)(r * row_stride + c * 16), slot_a + jj * 1024);
      }
    }
  };
  auto issue_next = [&]() __attribute__((always_inline)) {
    const int64_t u = iu++;
    const int64_t f = s0 + (u >> 1);
    const uint32_t slot = (uint32_t)(u % R);
    lds_reads_done();  // the slot's (and query slot's) earlier readers have their data
    int size = Gm::kPlaneIns;
    const int64_t hk = ip % a.hkv;
    if ((u & 1) == 0) {
      bool new_pair = u == 0;
      if (f == ipre1) {
        ip = pair_of(f);
        ipre0 = pre_l[ip];
        ipre1 = pair_end(ip);
        new_pair = true;
      }
      const int64_t b = ip / a.hkv;
      const int64_t j = f - ipre0;
      bool bad = false;
      if (a.seq_rows > 0) {
        irow = b * a.seq_rows + j * kPageTokens;
        const int64_t left = a.seq_rows - j * kPageTokens;
        irows = left < kPageTokens ? left : kPageTokens;
      } else {
        int32_t pid = ld_const(a.table + b * a.tstride + j);
        bad = pid < 0 || pid >= a.num_pages;
        if (bad) {
          if (lane == 0) raise_err(a.err, MKV_DEVERR_PAGE);
          pid = 0;
        }
        irow = (int64_t)pid * kPageTokens;
        irows = kPageTokens;
        icached = SHARED && pid < a.shared_below;
      }
      const uint32_t bit = 1u << ((f - s0) & 31);
      badbits = bad ? (badbits | bit) : (badbits & ~bit);
      const int64_t hk2 = ip % a.hkv;
      if (new_pair) {
        const uint8_t* qb = a.q + (int64_t)ip * G * kRowBytes;
        const uint32_t qs = q_a + (iqn % Gm::kQSlots) * Gm::kQBytes;
        ++iqn;
#pragma unroll
        for (int jj = 0; jj < Gm::kQIns; ++jj)
          dma16(qb, (uint32_t)((jj * 1024 + lane * 16) % (G * kRowBytes)), qs + jj * 1024);
        size += Gm::kQIns;
      }
      issue_plane(a.k + (irow * a.hkv + hk2) * Gm::kCodeRow, unit_a + slot * Gm::kPlane);
      if constexpr (FP8) {
        dma4(sbase + (irow + st) * a.hkv + hk2, scale_a + slot * Gm::kScaleBytes);
        size += Gm::kScaleIns;
      }
    } else {
      issue_plane(a.v + (irow * a.hkv + hk) * Gm::kCodeRow, unit_a + slot * Gm::kPlane);
    }
    fifo |= (uint32_t)size << (4 * fifo_n);
    ++fifo_n;
    fifo_total += size;
  };
  // waits for the oldest unit in flight (its loads and every earlier one)
  auto wait_oldest = [&]() __attribute__((always_inline)) {
    const int younger = fifo_total - (int)(fifo & 15u);
    if constexpr (R == 2) {
      // at most one younger unit: a V plane, a K plane (+ scales), or that
      // with a pair's query rows
      constexpr int kK = Gm::kPlaneIns + Gm::kScaleIns;
      if (younger == 0) vm_wait_n<0>();
      else if (younger == Gm::kPlaneIns) vm_wait_n<Gm::kPlaneIns>();
      else if (younger == kK) vm_wait_n<kK>();
      else if (younger == kK + Gm::kQIns) vm_wait_n<kK + Gm::kQIns>();
      else vm_wait(younger);
    } else {
      vm_wait(younger);
    }
  };
  auto retire_and_refill = [&]() __attribute__((always_inline)) {
    fifo_total -= (int)(fifo & 15u);
    fifo >>= 4;
    --fifo_n;
    if (iu < nunits) issue_next();
  };
  for (int k = 0; k < R && iu < nunits; ++k) issue_next();

  // ---- the consume side
  int32_t cp = wpair >= 0 ? wpair : pair_of(s0);  // pair of the page being consumed
  int64_t cpre0 = pre_l[cp], cpre1 = pair_end(cp);
  int32_t clen = len_l[cp];
  uint32_t cqn = 0;                // pairs whose query rows were read
  u32x4 qb[8];
  float m_run = -INFINITY, l_run = 0.f;  // head n (lanes n < G)
  float o[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] = 0.f;
  bool seg_first = true;

  for (int64_t f = s0; f < s1; ++f) {
    const int64_t uk = 2 * (f - s0);
    const uint32_t kslot = unit_a + (uint32_t)(uk % R) * Gm::kPlane;
    const uint32_t sslot = scale_a + (uint32_t)(uk % R) * Gm::kScaleBytes;
    const uint32_t vslot = unit_a + (uint32_t)((uk + 1) % R) * Gm::kPlane;
    __builtin_amdgcn_s_setprio(0);
    if ((((uint32_t)(f - s0) & 1u) ^ wslot) != 0) __builtin_amdgcn_s_setprio(1);
    // K plane (and query rows, scales) of page f
    wait_oldest();
    if (seg_first) {
      // the pair's query heads as the B operand, in the K operand's dim
      // order: bf16, step s covers dims 8*(4s+g) .. +7; fp8, K chunk 4r+g
      // holds 16 codes, step s = 2r+h covers dims 16*(4r+g) + 8h .. +7
      const uint32_t qs = q_a + (cqn % Gm::kQSlots) * Gm::kQBytes;
      ++cqn;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int chunk = FP8 ? 8 * (s >> 1) + 2 * g + (s & 1) : 4 * s + g;
        const u32x4 w = lds_ld16(qs + (n < G ? n : 0) * kRowBytes + chunk * 16);
        qb[s] = n < G ? w : u32x4{0u, 0u, 0u, 0u};
      }
    }
    // the page's K operand rows (and scales) into registers; the K slot is
    // then free and the ring is refilled before the MFMAs run
    u32x4 kr[FP8 ? 4 : 8];
#pragma unroll
    for (int s = 0; s < (FP8 ? 4 : 8); ++s) kr[s] = lds_ld16(kslot + koff[s]);
    float ksc[4], vsc[4];
    if constexpr (FP8) {
      const u32x4 kw = lds_ld16(sslot + 16 * g);
      const u32x4 vw = lds_ld16(sslot + 64 + 16 * g);
      ksc[0] = bits_f32(kw.x); ksc[1] = bits_f32(kw.y); ksc[2] = bits_f32(kw.z); ksc[3] = bits_f32(kw.w);
      vsc[0] = bits_f32(vw.x); vsc[1] = bits_f32(vw.y); vsc[2] = bits_f32(vw.z); vsc[3] = bits_f32(vw.w);
    }
    // page f's tokens of its pair: valid rows (0 for a page id outside the pool)
    const int64_t tok0 = (f - cpre0) * kPageTokens;
    const bool cbad = (badbits >> ((f - s0) & 31)) & 1u;
    const int valid = cbad ? 0 : (int)(clen - tok0 < kPageTokens ? clen - tok0 : kPageTokens);
    const bool seg_last = f + 1 == cpre1 || f + 1 == s1;
    retire_and_refill();
    f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (FP8) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc = mfma16<false>(fp8x8_bf16(kr[r].x, kr[r].y), qb[2 * r], sc);
        sc = mfma16<false>(fp8x8_bf16(kr[r].z, kr[r].w), qb[2 * r + 1], sc);
      }
    } else {
#pragma unroll
      for (int s = 0; s < 8; ++s) sc = mfma16<F16>(kr[s], qb[s], sc);
    }

    // online softmax for head n over the page's tokens 4g + i
    float sv[4], pm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float score = FP8 ? sc[i] * ksc[i] : sc[i];
      sv[i] = 4 * g + i < valid ? score * a.scale_log2 : -INFINITY;
      pm = fmaxf(pm, sv[i]);
    }
    pm = fmaxf(pm, __shfl_xor(pm, 16));
    pm = fmaxf(pm, __shfl_xor(pm, 32));
    const float m_new = fmaxf(m_run, pm);
    // -inf only while every token so far was masked: exponents stay -inf
    const float m_ref = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2_fast(m_run - m_ref);
    const bool rescale = __ballot(n < G && m_new != m_run) != 0;
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float pv = exp2_fast(sv[i] - m_ref);
      ps += pv;
      if (n < G) ptile[(4 * g + i) * G + n] = FP8 ? (4 * g + i < valid ? pv * vsc[i] : 0.f) : pv;
    }
    ps += __shfl_xor(ps, 16);
    ps += __shfl_xor(ps, 32);
    l_run = l_run * alpha + ps;
    m_run = m_new;
    if (rescale) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float al = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), h));
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] *= al;
      }
    }

    // V plane of page f
    wait_oldest();
    if (valid < kPageTokens) {
      // rows past the sequence's end (or of a page id outside the pool) may
      // hold anything: zero them so that 0-weight rows add exact zeros
      for (int i = lane; i < (kPageTokens - valid) * Gm::kChunks; i += 64) {
        const int r = valid + i / Gm::kChunks;
        *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(
            vslot + (r * Gm::kChunks + (i % Gm::kChunks)) * 16) = u32x4{0u, 0u, 0u, 0u};
      }
    }
    wave_sync();  // the probability tile and zeroed rows before the reads below
    // the page's V rows into registers; the V slot is then free and the ring
    // is refilled before the FMAs run
    typedef typename std::conditional<FP8, u32x2, u32x4>::type VRow;
    VRow vr[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if constexpr (FP8)
        vr[k] = lds_ld8(vslot + voffr[k]);
      else
        vr[k] = lds_ld16(vslot + voffr[k]);
    }
    retire_and_refill();
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int t = 8 * hf + k;
      float vv[8];
      if constexpr (FP8) {
        const f32x2 a0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)vr[k].x, false);
        const f32x2 a1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)vr[k].x, true);
        const f32x2 a2 = __builtin_amdgcn_cvt_pk_f32_fp8((int)vr[k].y, false);
        const f32x2 a3 = __builtin_amdgcn_cvt_pk_f32_fp8((int)vr[k].y, true);
        vv[0] = a0.x; vv[1] = a0.y; vv[2] = a1.x; vv[3] = a1.y;
        vv[4] = a2.x; vv[5] = a2.y; vv[6] = a3.x; vv[7] = a3.y;
      } else {
        const uint32_t ww[4] = {vr[k].x, vr[k].y, vr[k].z, vr[k].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vv[2 * e] = F16 ? f16_lo(ww[e]) : bf16_lo(ww[e]);
          vv[2 * e + 1] = F16 ? f16_hi(ww[e]) : bf16_hi(ww[e]);
        }
      }
      float pt[G];
      if constexpr (G >= 4) {
#pragma unroll
        for (int h4 = 0; h4 < G; h4 += 4) {
          const f32x4 p4 = *reinterpret_cast<const f32x4*>(&ptile[t * G + h4]);
          pt[h4] = p4[0]; pt[h4 + 1] = p4[1]; pt[h4 + 2] = p4[2]; pt[h4 + 3] = p4[3];
        }
      } else {
#pragma unroll
        for (int h = 0; h < G; ++h) pt[h] = ptile[t * G + h];
      }
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] += pt[h] * vv[e];
    }
    wave_sync();  // the next page rewrites the probability tile

    if (seg_last) {
      // the two token halves of the page hold the same dims: sum them
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] += __shfl_xor(o[h][e], 32);
      const bool whole = cpre0 >= s0 && cpre1 <= s1;
      if (whole) {
        uint8_t* orow = a.out + (int64_t)cp * G * kRowBytes;
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const float L = __builtin_bit_cast(
              float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l_run), h));
          if (hf == 0) {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
              w[e] = (uint32_t)out_bits<F16>(L > 0.f ? o[h][2 * e] / L : 0.f) |
                     ((uint32_t)out_bits<F16>(L > 0.f ? o[h][2 * e + 1] / L : 0.f) << 16);
            st16(orow + h * kRowBytes + c8 * 16, u32x4{w[0], w[1], w[2], w[3]});
          }
        }
      } else {
        // a piece of a pair cut by span boundaries: the span's first pair
        // goes to slot 0, its last pair to slot 1
        const int64_t at = (gw * 2 + (cpre0 <= s0 ? 0 : 1)) * G;
        if (hf == 0) {
#pragma unroll
          for (int h = 0; h < G; ++h) {
            float* pr = a.part + (at + h) * kHeadDim + 8 * c8;
            *reinterpret_cast<f32x4*>(pr) = f32x4{o[h][0], o[h][1], o[h][2], o[h][3]};
            *reinterpret_cast<f32x4*>(pr + 4) = f32x4{o[h][4], o[h][5], o[h][6], o[h][7]};
          }
        }
        if (lane < G) {
          a.ml[(at + lane) * 2] = m_run;
          a.ml[(at + lane) * 2 + 1] = l_run;
        }
      }
      m_run = -INFINITY;
      l_run = 0.f;
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] = 0.f;
      if (f + 1 < s1) {  // the next pair with pages
        cp = pair_of(f + 1);
        cpre0 = pre_l[cp];
        cpre1 = pair_end(cp);
        clen = len_l[cp];
      }
    }
    seg_first = seg_last;
  }
}

// Merges the pieces of one (pair, query head) of a pair cut by span
// boundaries, and writes the zeros of an empty pair. Every load of a batch
// of pieces is issued before the first is used (a loop with a remainder
// issued its last n % 8 loads a round trip apiece):
// - at most kMergeExact pieces (most cut pairs): a thread per dim, exactly
//   n pieces in one batch;
// - more (the longest pairs, 43 pieces at batch 256, which set the launch's
//   time): the pieces are dealt to the four waves (piece i to wave i % 4); a
//   wave keeps a running (max, sum, output) over batches of kMergeBatch, four
//   dims a lane, its (max, sum) pairs by one load broadcast by v_readlane,
//   and the waves' results are combined through LDS, a thread per dim. An
//   index past the last piece re-reads the last one and adds 0 x -0 (x + -0
//   is x for every x).
// The kernel stays at 44 VGPRs: the merge runs beside the prefill attention
// in the serving step, and forms of 52-76 VGPRs (more pieces a batch, the
// wave index not uniform) made the prefix-reuse serving step 1.7-2.6 %
// slower while their merges were faster.
constexpr int kMergeBatch = 4;   // pieces a wave loads at once (more pieces)
constexpr int kMergeExact = 16;  // pieces merged by one thread per dim in one batch

// The merge of a pair with exactly N pieces, a thread per dim: every load is
// issued before the first is used, the maximum is the pieces', and the sums
// run in piece order. Returns this thread's output value.
template <int N, typename AtOf>
__device__ __forceinline__ float merge_exact(const AttnArgs& a, AtOf at_of, int tid) {
  float m[N], l[N], p[N];
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const int64_t at = at_of(u);
    m[u] = ld_const(a.ml + at * 2);
    l[u] = ld_const(a.ml + at * 2 + 1);
    p[u] = a.part[at * kHeadDim + tid];
  }
  float M = -INFINITY;
#pragma unroll
  for (int u = 0; u < N; ++u) M = fmaxf(M, m[u]);
  float O = 0.f, L = 0.f;
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const float f = m[u] == -INFINITY ? 0.f : exp2_fast(m[u] - M);
    O += f * p[u];
    L += f * l[u];
  }
  return L > 0.f ? O / L : 0.f;
}

template <int G, bool F16>
__global__ __launch_bounds__(kAttnThreads) void attn_merge_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) float wave_o[kAttnWaves][kHeadDim];
  __shared__ float wave_ml[kAttnWaves][2];
  const int64_t pr = blockIdx.x / G;
  const int h = blockIdx.x % G;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: piece addresses in SGPRs
  // the span is loaded with the pair's bounds (the empty asm keeps the
  // compiler from moving its load behind the branch below)
  const int64_t span = ld_const(a.hdr);
  const int32_t p0 = ld_const(a.pre + pr), p1 = ld_const(a.pend + pr);
  asm volatile("" ::"s"(span));
  uint8_t* out = a.out + (pr * G + h) * kRowBytes;
  if (p1 <= p0) {  // nothing to attend to: zeros
    reinterpret_cast<uint16_t*>(out)[tid] = 0;
    return;
  }
  // flat page indices are int32, and the span is at most the launch's pages
  const uint32_t S = (uint32_t)span;
  const uint32_t w0 = (uint32_t)p0 / S, w1 = (uint32_t)(p1 - 1) / S;
  if (w0 == w1) return;  // written by its wave
  const int n_seg = (int)(w1 - w0 + 1);
  // piece i: wave w0 + i, slot 1 for the first piece unless the pair starts
  // its span (then it is that span's first pair), slot 0 for the rest
  auto at_of = [&](int i) __attribute__((always_inline)) {
    const int64_t w = (int64_t)w0 + i;
    const int slot = (i == 0 && (uint32_t)p0 != w0 * S) ? 1 : 0;
    return (w * 2 + slot) * G + h;
  };
  if (n_seg <= kMergeExact) {  // most cut pairs: one round trip, no duplicate loads
    float r;
    switch (n_seg) {
      case 2: r = merge_exact<2>(a, at_of, tid); break;
      case 3: r = merge_exact<3>(a, at_of, tid); break;
      case 4: r = merge_exact<4>(a, at_of, tid); break;
      case 5: r = merge_exact<5>(a, at_of, tid); break;
      case 6: r = merge_exact<6>(a, at_of, tid); break;
      case 7: r = merge_exact<7>(a, at_of, tid); break;
      case 8: r = merge_exact<8>(a, at_of, tid); break;
      case 9: r = merge_exact<9>(a, at_of, tid); break;
      case 10: r = merge_exact<10>(a, at_of, tid); break;
      case 11: r = merge_exact<11>(a, at_of, tid); break;
      case 12: r = merge_exact<12>(a, at_of, tid); break;
      case 13: r = merge_exact<13>(a, at_of, tid); break;
      case 14: r = merge_exact<14>(a, at_of, tid); break;
      case 15: r = merge_exact<15>(a, at_of, tid); break;
      default: r = merge_exact<16>(a, at_of, tid); break;
    }
    reinterpret_cast<uint16_t*>(out)[tid] = out_bits<F16>(r);
    return;
  }
  float m_run = -INFINITY, l_run = 0.f;
  f32x4 o_run = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int i0 = wave; i0 < n_seg; i0 += kAttnWaves * kMergeBatch) {
    const int mine = i0 + kAttnWaves * (lane & (kMergeBatch - 1));
    const float2 ml =
        *reinterpret_cast<const float2*>(a.ml + at_of(mine < n_seg ? mine : n_seg - 1) * 2);
    f32x4 p[kMergeBatch];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const int i = i0 + kAttnWaves * u;
      p[u] = *reinterpret_cast<const f32x4*>(a.part + at_of(i < n_seg ? i : n_seg - 1) * kHeadDim +
                                             4 * lane);
    }
    float m[kMergeBatch], l[kMergeBatch];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      m[u] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ml.x), u));
      l[u] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ml.y), u));
    }
    float mb = m_run;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u)
      mb = fmaxf(mb, i0 + kAttnWaves * u < n_seg ? m[u] : -INFINITY);
    // mb >= m_run; a wave's first batch starts from nothing
    const float alpha = m_run == -INFINITY ? 0.f : exp2_fast(m_run - mb);
    l_run *= alpha;
    o_run *= alpha;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const bool ok = i0 + kAttnWaves * u < n_seg;
      const float f = !ok || m[u] == -INFINITY ? 0.f : exp2_fast(m[u] - mb);
#pragma unroll
      for (int e = 0; e < 4; ++e) o_run[e] += f * (ok ? p[u][e] : -0.f);
      l_run += f * (ok ? l[u] : -0.f);
    }
    m_run = mb;
  }
  *reinterpret_cast<f32x4*>(&wave_o[wave][4 * lane]) = o_run;
  if (lane == 0) {
    wave_ml[wave][0] = m_run;
    wave_ml[wave][1] = l_run;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, wave_ml[w][0]);
  float O = 0.f, L = 0.f;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) {
    const float mw = wave_ml[w][0];
    const float f = mw == -INFINITY ? 0.f : exp2_fast(mw - M);
    O += f * wave_o[w][tid];
    L += f * wave_ml[w][1];
  }
  reinterpret_cast<uint16_t*>(out)[tid] = out_bits<F16>(L > 0.f ? O / L : 0.f);
}

// Workgroups of the span kernel: as many as are resident at once (CUs x the
// kernel's occupancy at this launch's LDS size), so every wave's span starts
// at once. The occupancy depends on the pair count only through the LDS
// size; it is looked up once per (device, kernel, pair count).
std::mutex g_grid_mu;
struct GridKey {
  int dev, kind, G, pairs;
  bool operator==(const GridKey& o) const {
    return dev == o.dev && kind == o.kind && G == o.G && pairs == o.pairs;
  }
};
constexpr int kGridMemo = 64;
GridKey g_grid_key[kGridMemo];
int g_grid_val[kGridMemo];
int g_grid_n = 0;

// Workgroups per CU that this launch's LDS allows (at most 4): an upper
// bound of the kernel's occupancy computable on the host alone, which sizes
// the workspace.
template <int G, bool FP8>
int occ_cap(int32_t pairs) {
  const int by_lds = (int)(kLdsPerCu / attn_lds_bytes<G, FP8>(pairs));
  return by_lds < 4 ? (by_lds < 1 ? 1 : by_lds) : 4;
}

// CUs of the current device (256, MI355X's count, when none can be queried).
int device_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    return 256;
  return n;
}

template <int G, bool FP8, bool F16>
int attn_grid(int kind, int32_t pairs) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  const GridKey key{dev, kind, G, pairs};
  {
    std::lock_guard<std::mutex> lock(g_grid_mu);
    for (int i = 0; i < g_grid_n; ++i)
      if (g_grid_key[i] == key) return g_grid_val[i];
  }
  // the slots of four waves need more than the default 64 KiB of dynamic LDS
  // (the attribute is per kernel and device; it must be set before the
  // occupancy query, which honours it)
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(attn_span_kernel<G, FP8, F16, false>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, 159 * 1024) != hipSuccess ||
      hipFuncSetAttribute(reinterpret_cast<const void*>(attn_span_kernel<G, FP8, F16, true>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, 159 * 1024) != hipSuccess)
    return -1;
  int per = 0;
  const size_t lds = attn_lds_bytes<G, FP8>(pairs);
  // the grid of the variant without shared pages (the other one has at least
  // as many registers; the launch checks its own occupancy below)
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, attn_span_kernel<G, FP8, F16, false>,
                                                   kAttnThreads, lds) != hipSuccess ||
      per <= 0)
    per = 1;
  const int cap = occ_cap<G, FP8>(pairs);
  const int grid = device_cus() * (per < cap ? per : cap);
  std::lock_guard<std::mutex> lock(g_grid_mu);
  const int slot = g_grid_n < kGridMemo ? g_grid_n++ : (int)((unsigned)pairs % kGridMemo);
  g_grid_key[slot] = key;
  g_grid_val[slot] = grid;
  return grid;
}

template <int G, bool FP8, bool F16>
int launch_attn(AttnArgs a, int grid, hipStream_t st) {
  const size_t lds = attn_lds_bytes<G, FP8>(a.pairs);
  if (a.shared_below > 0)
    hipLaunchKernelGGL((attn_span_kernel<G, FP8, F16, true>), dim3((unsigned)grid),
                       dim3(kAttnThreads), lds, st, a);
  else
    hipLaunchKernelGGL((attn_span_kernel<G, FP8, F16, false>), dim3((unsigned)grid),
                       dim3(kAttnThreads), lds, st, a);
  hipLaunchKernelGGL((attn_merge_kernel<G, F16>), dim3((unsigned)(a.pairs * G)),
                     dim3(kAttnThreads), 0, st, a);
  return MKV_OK;
}

// Element kinds of the pool the entry points read.
enum AttnKind { kAttnBf16, kAttnFp8, kAttnF16 };

template <int G>
int grid_of(AttnKind kind, int32_t pairs) {
  if (kind == kAttnFp8) return attn_grid<G, true, false>(kind, pairs);
  if (kind == kAttnF16) return attn_grid<G, false, true>(kind, pairs);
  return attn_grid<G, false, false>(kind, pairs);
}

// The span kernel's grid for a kind, G and pair count (cached per device).
int span_grid(AttnKind kind, int32_t G, int32_t pairs) {
  switch (G) {
    case 1: return grid_of<1>(kind, pairs);
    case 2: return grid_of<2>(kind, pairs);
    case 4: return grid_of<4>(kind, pairs);
    default: return grid_of<8>(kind, pairs);
  }
}

// Workspace layout: header, pairs' flat starts and ends, piece (max, sum),
// piece outputs.
struct WsLayout {
  int64_t pre, pend, ml, part, total;
};
inline WsLayout ws_layout(int64_t pairs, int64_t G, int64_t waves) {
  WsLayout w;
  w.pre = kHeaderBytes;
  w.pend = w.pre + ((pairs + 1) * 4 + 255) / 256 * 256;
  w.ml = w.pend + (pairs * 4 + 255) / 256 * 256;
  w.part = w.ml + (waves * 2 * G * 2 * 4 + 255) / 256 * 256;
  w.total = w.part + waves * 2 * G * kHeadDim * 4;
  return w;
}

// Waves of the largest grid a kind's launch can use for this G and pair
// count (the CUs times the LDS-bound occupancy); host-only, so the workspace
// can be sized without a device.
template <int G>
int64_t kind_waves(AttnKind kind, int32_t pairs) {
  const int cap = kind == kAttnFp8 ? occ_cap<G, true>(pairs) : occ_cap<G, false>(pairs);
  return (int64_t)device_cus() * cap * kAttnWaves;
}
int64_t bound_waves(AttnKind kind, int32_t G, int32_t pairs) {
  switch (G) {
    case 1: return kind_waves<1>(kind, pairs);
    case 2: return kind_waves<2>(kind, pairs);
    case 4: return kind_waves<4>(kind, pairs);
    default: return kind_waves<8>(kind, pairs);
  }
}

// Workspace bytes a launch over one pool kind needs at most.
int64_t kind_workspace_bytes(AttnKind kind, int32_t batch, int32_t num_kv_heads,
                             int32_t num_q_heads) {
  if (batch < 0 || num_kv_heads <= 0 || num_q_heads <= 0) return -1;
  const int32_t G = num_q_heads / num_kv_heads;
  if (G * num_kv_heads != num_q_heads || !(G == 1 || G == 2 || G == 4 || G == 8)) return -1;
  const int64_t pairs = (int64_t)batch * num_kv_heads;
  if (pairs > kMaxPairs) return -1;
  return ws_layout(pairs, G, bound_waves(kind, G, (int32_t)pairs)).total;
}

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int64_t mkv_decode_attention_workspace_bytes(int32_t batch, int32_t num_kv_heads,
                                                        int32_t num_q_heads, int32_t max_seq_len) {
  if (max_seq_len < 0) return -1;
  int64_t best = -1;
  for (AttnKind k : {kAttnBf16, kAttnFp8, kAttnF16}) {
    const int64_t n = kind_workspace_bytes(k, batch, num_kv_heads, num_q_heads);
    if (n < 0) return -1;
    if (n > best) best = n;
  }
  return best;
}

namespace {

template <int G>
int launch_kind(AttnKind kind, const AttnArgs& a, int grid, hipStream_t st) {
  if (kind == kAttnFp8) return launch_attn<G, true, false>(a, grid, st);
  if (kind == kAttnF16) return launch_attn<G, false, true>(a, grid, st);
  return launch_attn<G, false, false>(a, grid, st);
}

// Shared by the entry points: `fn` names the caller in error messages; the
// scale planes are null for 16-bit caches; seq_rows > 0 selects contiguous
// caches [batch, seq_rows, num_kv_heads, 256] (no page table).
int decode_attention(const char* fn, AttnKind kind, const void* q, const void* k_cache,
                     const void* v_cache, const float* k_scales, const float* v_scales,
                     int64_t num_pages, int64_t shared_pages, int32_t num_kv_heads, int32_t num_q_heads,
                     int32_t head_dim, const int32_t* page_table, int64_t table_stride,
                     int32_t table_width, int64_t seq_rows, const int32_t* seq_lens,
                     int32_t batch, int32_t max_seq_len, float softmax_scale, void* out,
                     void* workspace, int64_t workspace_bytes, int32_t* err, void* stream) {
  clear_error();
  MKV_REQUIRE(batch >= 0 && num_pages > 0 && num_kv_heads > 0 && num_q_heads > 0 &&
                  table_width >= 0 && table_stride >= table_width && max_seq_len >= 0 &&
                  shared_pages >= 0,
              MKV_E_INVALID, "%s: bad sizes", fn);
  MKV_REQUIRE(head_dim == kHeadDim, MKV_E_UNSUPPORTED, "%s: head_dim %d unsupported (256)", fn,
              head_dim);
  const int32_t G = num_q_heads / num_kv_heads;
  MKV_REQUIRE(G * num_kv_heads == num_q_heads && (G == 1 || G == 2 || G == 4 || G == 8),
              MKV_E_UNSUPPORTED, "%s: %d query heads per KV head unsupported (1, 2, 4, 8)", fn,
              num_q_heads / num_kv_heads);
  if (batch == 0) return MKV_OK;
  MKV_REQUIRE(q && k_cache && v_cache && (seq_rows > 0 || page_table) && seq_lens && out && err &&
                  (kind != kAttnFp8 || (k_scales && v_scales)),
              MKV_E_INVALID, "%s: null pointer", fn);
  MKV_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out),
              MKV_E_ALIGN, "%s: q, caches and out must be 16-byte aligned", fn);
  MKV_REQUIRE(kind != kAttnFp8 || (aligned4(k_scales) && aligned4(v_scales)), MKV_E_ALIGN,
              "%s: scale planes must be 4-byte aligned", fn);
  MKV_REQUIRE((int64_t)batch * num_kv_heads <= kMaxPairs, MKV_E_UNSUPPORTED,
              "%s: batch x KV heads above %d", fn, kMaxPairs);
  MKV_REQUIRE(max_seq_len <= (1 << 24), MKV_E_UNSUPPORTED, "%s: max_seq_len above 2^24", fn);
  // the pages of all pairs are counted in 32 bits
  MKV_REQUIRE((int64_t)batch * num_kv_heads * (((int64_t)max_seq_len + 15) / 16) < (1ll << 31),
              MKV_E_UNSUPPORTED, "%s: batch x KV heads x pages above 2^31", fn);
  const int32_t pairs = batch * num_kv_heads;
  const int grid = span_grid(kind, G, pairs);
  MKV_REQUIRE(grid > 0, MKV_E_LAUNCH, "%s: cannot size the grid (dynamic LDS attribute)", fn);
  const WsLayout L = ws_layout(pairs, G, (int64_t)grid * kAttnWaves);
  MKV_REQUIRE(workspace && workspace_bytes >= L.total && aligned16(workspace), MKV_E_INVALID,
              "%s: workspace of %lld bytes (16-byte aligned) required", fn, (long long)L.total);
  AttnArgs a;
  a.q = static_cast<const uint8_t*>(q);
  a.k = static_cast<const uint8_t*>(k_cache);
  a.v = static_cast<const uint8_t*>(v_cache);
  a.ks = k_scales;
  a.vs = v_scales;
  a.table = page_table;
  a.lens = seq_lens;
  a.out = static_cast<uint8_t*>(out);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  a.hdr = reinterpret_cast<int64_t*>(ws);
  a.pre = reinterpret_cast<int32_t*>(ws + L.pre);
  a.pend = reinterpret_cast<int32_t*>(ws + L.pend);
  a.ml = reinterpret_cast<float*>(ws + L.ml);
  a.part = reinterpret_cast<float*>(ws + L.part);
  a.num_pages = num_pages;
  a.shared_below = shared_pages;
  a.tstride = table_stride;
  a.seq_rows = seq_rows;
  a.twidth = table_width;
  a.hkv = num_kv_heads;
  a.max_len = max_seq_len;
  a.pairs = pairs;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.err = err;
  const hipStream_t st = as_stream(stream);
  int rc;
  switch (G) {
    case 1: rc = launch_kind<1>(kind, a, grid, st); break;
    case 2: rc = launch_kind<2>(kind, a, grid, st); break;
    case 4: rc = launch_kind<4>(kind, a, grid, st); break;
    default: rc = launch_kind<8>(kind, a, grid, st); break;
  }
  if (rc != MKV_OK) return rc;
  return check_launch(fn);
}

}  // namespace

extern "C" int mkv_decode_attention_bf16(const void* q, const void* k_cache, const void* v_cache,
                                         int64_t num_pages, int64_t shared_pages,
                                         int32_t num_kv_heads, int32_t num_q_heads,
                                         int32_t head_dim, const int32_t* page_table,
                                         int64_t table_stride, int32_t table_width,
                                         const int32_t* seq_lens, int32_t batch,
                                         int32_t max_seq_len, float softmax_scale, void* out,
                                         void* workspace, int64_t workspace_bytes, int32_t* err,
                                         void* stream) {
  return decode_attention("mkv_decode_attention_bf16", kAttnBf16, q, k_cache, v_cache, nullptr,
                          nullptr, num_pages, shared_pages, num_kv_heads, num_q_heads, head_dim,
                          page_table, table_stride, table_width, 0, seq_lens, batch, max_seq_len,
                          softmax_scale, out, workspace, workspace_bytes, err, stream);
}

extern "C" int mkv_decode_attention_fp8(const void* q, const void* k_codes, const void* v_codes,
                                        const float* k_scales, const float* v_scales,
                                        int64_t num_pages, int64_t shared_pages,
                                        int32_t num_kv_heads, int32_t num_q_heads,
                                        int32_t head_dim, const int32_t* page_table,
                                        int64_t table_stride, int32_t table_width,
                                        const int32_t* seq_lens, int32_t batch,
                                        int32_t max_seq_len, float softmax_scale, void* out,
                                        void* workspace, int64_t workspace_bytes, int32_t* err,
                                        void* stream) {
  return decode_attention("mkv_decode_attention_fp8", kAttnFp8, q, k_codes, v_codes, k_scales,
                          v_scales, num_pages, shared_pages, num_kv_heads, num_q_heads, head_dim,
                          page_table, table_stride, table_width, 0, seq_lens, batch, max_seq_len,
                          softmax_scale, out, workspace, workspace_bytes, err, stream);
}

extern "C" int mkv_decode_attention_f16(const void* q, const void* k_cache, const void* v_cache,
                                        int64_t num_pages, int64_t shared_pages,
                                        int32_t num_kv_heads, int32_t num_q_heads,
                                        int32_t head_dim, const int32_t* page_table,
                                        int64_t table_stride, int32_t table_width,
                                        const int32_t* seq_lens, int32_t batch,
                                        int32_t max_seq_len, float softmax_scale, void* out,
                                        void* workspace, int64_t workspace_bytes, int32_t* err,
                                        void* stream) {
  return decode_attention("mkv_decode_attention_f16", kAttnF16, q, k_cache, v_cache, nullptr,
                          nullptr, num_pages, shared_pages, num_kv_heads, num_q_heads, head_dim,
                          page_table, table_stride, table_width, 0, seq_lens, batch, max_seq_len,
                          softmax_scale, out, workspace, workspace_bytes, err, stream);
}

extern "C" int mkv_decode_attention_contig(const void* q, const void* k_cache,
                                           const void* v_cache, int32_t fp16,
                                           int32_t num_kv_heads, int32_t num_q_heads,
                                           int32_t head_dim, int64_t seq_rows,
                                           const int32_t* seq_lens, int32_t batch,
                                           int32_t max_seq_len, float softmax_scale, void* out,
                                           void* workspace, int64_t workspace_bytes,
                                           int32_t* err, void* stream) {
  static const char* fn = "mkv_decode_attention_contig";
  clear_error();
  MKV_REQUIRE(seq_rows > 0 && (int64_t)batch * seq_rows < (1ll << 40), MKV_E_INVALID,
              "%s: seq_rows must be positive", fn);
  // lengths are cut to the rows each sequence owns (MKV_DEVERR_TABLE past them)
  const int64_t pages = (seq_rows + 15) / 16;
  MKV_REQUIRE(pages <= INT32_MAX, MKV_E_UNSUPPORTED, "%s: seq_rows too large", fn);
  const int32_t cap = max_seq_len < seq_rows ? max_seq_len : (int32_t)seq_rows;
  return decode_attention(fn, fp16 ? kAttnF16 : kAttnBf16, q, k_cache, v_cache, nullptr, nullptr,
                          (int64_t)batch * pages, 0, num_kv_heads, num_q_heads, head_dim, nullptr,
                          pages, (int32_t)pages, seq_rows, seq_lens, batch, cap, softmax_scale,
                          out, workspace, workspace_bytes, err, stream);
}

// ---------------------------------------------------------------------------
// The same bf16 decode attention for callers that cannot allocate (code under
// HIP graph capture, tight serving loops): the workspace is a file-scope
// device array, one copy per GPU, held until the process ends.
// ---------------------------------------------------------------------------
namespace {

// Room for the header, the page prefix of up to 4096 pairs and the pieces of
// every resident wave (2048 waves x 2 pieces x 4 query heads x 1032 bytes at
// four query heads per KV head on MI355X: 17 MB).
constexpr int64_t kNoAllocScratchBytes = 48ll << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The current device's copy of `scratch`. In host code the array's name is
// only a stand-in for the symbol: its device address comes from
// hipGetSymbolAddress, once per device (with that device current), and only
// that address is ever handed to a kernel. Nothing in it needs to start at
// zero: every call writes the header and prefix before the pieces are read.
int scratch_of_current_device(const char* fn, void** out) {
  int dev = -1;
  const hipError_t ge = hipGetDevice(&dev);
  if (ge != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return set_error(MKV_E_LAUNCH, "%s: no usable current device (%s)", fn,
                     ge != hipSuccess ? hipGetErrorString(ge) : "device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(MKV_E_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed: %s", fn,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MKV_OK;
}

}  // namespace

extern "C" int mkv_decode_attention_bf16_noalloc(const void* q, const void* k_cache,
                                                 const void* v_cache, int64_t num_pages,
                                                 int32_t num_kv_heads, int32_t num_q_heads,
                                                 int32_t head_dim, const int32_t* page_table,
                                                 int64_t table_stride, int32_t table_width,
                                                 const int32_t* seq_lens, int32_t batch,
                                                 int32_t max_seq_len, float softmax_scale,
                                                 void* out, int32_t* err, void* stream) {
  static const char* fn = "mkv_decode_attention_bf16_noalloc";
  clear_error();
  const int64_t need = max_seq_len < 0 ? -1
                                        : kind_workspace_bytes(kAttnBf16, batch, num_kv_heads,
                                                               num_q_heads);
  MKV_REQUIRE(need >= 0, MKV_E_UNSUPPORTED, "%s: unsupported shape (batch %d, %d KV heads, %d "
              "query heads)", fn, batch, num_kv_heads, num_q_heads);
  MKV_REQUIRE(need <= kNoAllocScratchBytes, MKV_E_UNSUPPORTED,
              "%s: batch %d x %d query heads need %lld bytes of scratch, the static scratch "
              "holds %lld", fn, batch, num_q_heads, (long long)need,
              (long long)kNoAllocScratchBytes);
  if (batch == 0) return decode_attention(fn, kAttnBf16, q, k_cache, v_cache, nullptr, nullptr,
                                          num_pages, 0, num_kv_heads, num_q_heads, head_dim,
                                          page_table, table_stride, table_width, 0, seq_lens,
                                          batch, max_seq_len, softmax_scale, out, nullptr, 0,
                                          err, stream);
  void* ws = nullptr;
  const int rc = scratch_of_current_device(fn, &ws);
  if (rc != MKV_OK) return rc;
  return decode_attention(fn, kAttnBf16, q, k_cache, v_cache, nullptr, nullptr, num_pages, 0,
                          num_kv_heads, num_q_heads, head_dim, page_table, table_stride,
                          table_width, 0, seq_lens, batch, max_seq_len, softmax_scale, out, ws,
                          kNoAllocScratchBytes, err, stream);
}
