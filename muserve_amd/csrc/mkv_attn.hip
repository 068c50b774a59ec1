// mkv_attn.hip — paged decode attention reading the KV pool directly (gfx950).
//
// One decode query token per sequence attends to the first seq_lens[b] cached
// tokens of its block table: for each of the G query heads sharing a KV head,
// softmax(q k^T * scale) v over the sequence, computed in fp32, written as
// bf16. This is the interface of the paged decode kernel the reference wraps
// (muserve/kernels/attention.py:29-42) and the math of its contiguous decode
// path (muserve/model/qwen35_layer_v2.py:493-502), without the padded gather.
//
// Each K/V row is read once, 4 flop per byte at G = 4, so the bound is HBM.
// A workgroup (4 waves) takes a 1024-token chunk of one sequence and KV head;
// a wave takes one 16-token page at a time:
//   * scores on MFMA (v_mfma_f32_16x16x32_bf16, 8 steps over head_dim 256):
//     A = the K page, 16 contiguous bytes of a K row per lane loaded straight
//     from the pool (row = lane % 16, 16-byte chunk 4*step + lane / 16);
//     B = the G query heads (columns >= G zero) in the same dim order, held
//     in registers for the whole chunk; C = 4 scores per lane (tokens
//     4*(lane/16) + i, head lane % 16);
//   * online softmax per head in fp32 (exp2, log2(e) folded into the scale);
//     the page's probabilities go through a wave-private LDS tile;
//   * P V on the VALU: a lane owns dims 4*lane .. 4*lane+3 of all G heads, so
//     a V row is one coalesced 512-byte load per wave, with no transpose;
//   * the waves' partial softmax states merge in LDS. A one-chunk sequence
//     writes its normalised output; longer ones write (max, sum, unnormalised
//     output) per chunk to the caller's workspace and a second kernel merges
//     them, one workgroup per (sequence, query head).
// The chunks of all sequences form one list (sequence-major; every workgroup
// computes the prefix of the chunk counts in LDS) that a grid of a few
// workgroups per CU drains: the first item of each workgroup is its own
// index, the rest come from an atomic counter. No workgroup is launched for a
// chunk beyond its sequence's end, and the load balances whatever the
// lengths. The merge kernel, which runs next, resets the counter.
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

constexpr int kHeadDim = 256;
constexpr int kRowBytes = kHeadDim * 2;  // one bf16 K or V row of one KV head
constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr int kPageTokens = 16;
constexpr int kChunk = 1024;  // tokens per work item (512 measured 3 % slower, 2048 4 %)
constexpr int kChunkPages = kChunk / kPageTokens;
constexpr int kMaxPairs = 4096;  // batch x KV heads whose chunk prefix fits in LDS
constexpr int kPagesPerIter = 1;  // pages per wave iteration (2 measured 1.5 % slower on fp8)
constexpr int kIterTokens = kPagesPerIter * kPageTokens;
constexpr int kTailClasses = 32;  // length classes of the short chunks (32 tokens each)
constexpr int kTailNone = 255;    // a pair without a short chunk

struct AttnArgs {
  const uint8_t* q;  // [B, Hkv * G, 256] bf16
  const uint8_t* k;  // [P, 16, Hkv, 256] bf16, or e4m3fn codes
  const uint8_t* v;
  const float* ks;   // fp8 caches: [P, 16, Hkv] fp32 scales of K and V
  const float* vs;
  const int32_t* table;  // [B, tstride] int32
  const int32_t* lens;   // [B] int32
  uint8_t* out;          // [B, Hkv * G, 256] bf16
  float* part;           // [B, Hkv, chunks, G, 256] unnormalised chunk outputs
  float* ml;             // [B, Hkv, chunks, G, 2] chunk (max, sum), log2 units
  int32_t* queue;        // [1]: next dynamic work item (zero between calls)
  int64_t num_pages, tstride;
  int32_t twidth, hkv, chunks, max_len, pairs;
  float scale_log2;  // softmax_scale * log2(e)
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

// The sequence length the kernels use: clamped to what the table holds and
// to the launch's bound (MKV_DEVERR_TABLE when clamped), 0 if negative.
__device__ __forceinline__ int64_t attn_len(const AttnArgs& a, int64_t b, bool report) {
  int64_t len = ld_const(a.lens + b);
  const int64_t cap = (int64_t)a.twidth * kPageTokens < a.max_len
                          ? (int64_t)a.twidth * kPageTokens
                          : (int64_t)a.max_len;
  if (len > cap || len < 0) {
    if (report) raise_err(a.err, MKV_DEVERR_TABLE);
    len = len < 0 ? 0 : cap;
  }
  return len;
}

// Eight e4m3fn codes (little-endian bytes of lo, hi) as eight bf16: exact,
// every e4m3fn value is a bf16 value. gfx950 converts a code pair straight to
// a bf16 pair (v_cvt_scalef32_pk_bf16_fp8, scale 1): four instructions per
// eight codes instead of eight through fp32 (mkv_check_conversions checks it
// on every code).
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ bf16x8 fp8x8_bf16(uint32_t lo, uint32_t hi) {
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)lo, 1.0f, false);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)lo, 1.0f, true);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)hi, 1.0f, false);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)hi, 1.0f, true);
  return bf16x8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// One 1024-token chunk of one (sequence, KV head). FP8: the caches hold
// e4m3fn codes with an fp32 scale per (token, KV head); a token's score is
// scale_k * (q . codes) and its V weight p * scale_v, so the codes convert
// exactly to bf16 MFMA operands and no product is rounded before the fp32
// accumulation. F16: q, caches and out are fp16 instead of bf16.
template <int G, bool FP8, bool F16>
__device__ __forceinline__ void attn_chunk(const AttnArgs& a, int64_t b, int64_t hk, int64_t c,
                                           int64_t len, int64_t nch,
                                           float (&p_lds)[kAttnWaves][kIterTokens][16],
                                           float (&al_lds)[kAttnWaves][16],
                                           float (&m_w)[kAttnWaves][G], float (&l_w)[kAttnWaves][G],
                                           float (&o_w)[kAttnWaves][G][kHeadDim]) {
  constexpr int kCodeRow = FP8 ? kHeadDim : kRowBytes;  // bytes of one cached K or V row
  constexpr int PPI = kPagesPerIter;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar page ids
  const int n = lane & 15, g = lane >> 4;
  uint8_t* out = a.out + (b * a.hkv + hk) * G * kRowBytes;
  if (len == 0) {  // nothing to attend to: zeros
    for (int i = threadIdx.x; i < G * kRowBytes / 16; i += kAttnThreads)
      st16(out + i * 16, u32x4{0u, 0u, 0u, 0u});
    return;
  }

  // The G query heads as the B operand, in the K operand's dim order. Lane
  // group g loads the 16-byte chunks 4r+g of a K row (a load instruction reads
  // 64 contiguous bytes of each of the 16 rows): bf16, step s = r covers dims
  // 8*(4s+g) .. +7; fp8, a chunk holds 16 codes, step s = 2r+h covers dims
  // 16*(4r+g) + 8h .. +7, the q chunk 8r + 2g + h.
  u32x4 qb[8];
  const uint8_t* qrow = a.q + ((b * a.hkv + hk) * G + (n < G ? n : 0)) * kRowBytes;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const int chunk = FP8 ? 8 * (s >> 1) + 2 * g + (s & 1) : 4 * s + g;
    const u32x4 w = n < G ? ld16(qrow + chunk * 16) : u32x4{0u, 0u, 0u, 0u};
    qb[s] = w;
  }
  float m_run = -INFINITY, l_run = 0.f;  // head n
  float o[G][4];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int j = 0; j < 4; ++j) o[h][j] = 0.f;

  const int64_t tok_stride = (int64_t)a.hkv * kCodeRow;
  const int64_t pages = (len + kPageTokens - 1) / kPageTokens;
  const int64_t p_end = (c + 1) * (int64_t)kChunkPages < pages ? (c + 1) * (int64_t)kChunkPages : pages;
  const int32_t* trow = a.table + b * a.tstride;
  // This wave's pages are p0 + 4q, q < np: their ids in one load, lane q
  // holding page q. A page id outside the pool is flagged and its tokens
  // masked (page 0 is read in its place), so the loop below has no branches
  // and the compiler's load counting stays exact.
  static_assert(kChunkPages / kAttnWaves <= 32, "a wave's page validity fits a 32-bit mask");
  const int64_t p0 = c * (int64_t)kChunkPages + wave;
  const int np = p_end > p0 ? (int)((p_end - p0 + kAttnWaves - 1) / kAttnWaves) : 0;
  const int32_t pid_raw = lane < np ? trow[p0 + (int64_t)kAttnWaves * lane] : 0;
  const bool bad = lane < np && (pid_raw < 0 || pid_raw >= a.num_pages);
  const uint32_t badmask = (uint32_t)__ballot(bad);
  if (badmask && lane == 0) raise_err(a.err, MKV_DEVERR_PAGE);
  const int32_t pid_v = bad ? 0 : pid_raw;
  auto page_row = [&](int q) {  // page q's first (token, KV head) row; q >= np: page np-1
    return (int64_t)__builtin_amdgcn_readlane(pid_v, q < np ? q : np - 1) * kPageTokens * a.hkv +
           hk;
  };
  // Software pipeline over iterations of PPI pages: the next iteration's K
  // (and scales) are loaded once the score MFMAs have read this one's, and its
  // V rows one by one as P V consumes this one's, into the same registers.
  // Past the wave's last page the loads repeat that page (cache hits) and the
  // tokens are masked.
  typedef u32x4 KReg;
  typedef typename std::conditional<FP8, uint32_t, u32x2>::type VReg;
  constexpr int kKRegs = FP8 ? 4 : 8;
  KReg ka[PPI][kKRegs];
  VReg vr[PPI][kPageTokens];
  float sk[PPI][4], svs[PPI][4];  // fp8: scales of tokens 4g+i
  auto load_k = [&](int u, int64_t row) {
    const uint8_t* kp = a.k + row * kCodeRow + n * tok_stride;
    if constexpr (FP8) {
#pragma unroll
      for (int r = 0; r < 4; ++r) ka[u][r] = ld16(kp + 16 * (4 * r + g));
      // (one load and shuffles instead: 1 % faster, 18 more VGPRs)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sk[u][i] = a.ks[row + (int64_t)(4 * g + i) * a.hkv];
        svs[u][i] = a.vs[row + (int64_t)(4 * g + i) * a.hkv];
      }
    } else {
#pragma unroll
      for (int s = 0; s < 8; ++s) ka[u][s] = ld16(kp + (4 * s + g) * 16);
    }
  };
  auto load_v = [&](int u, int64_t row, int t) {
    const uint8_t* vp = a.v + row * kCodeRow + t * tok_stride;
    if constexpr (FP8)
      vr[u][t] = *reinterpret_cast<const uint32_t*>(vp + lane * 4);
    else
      vr[u][t] = *reinterpret_cast<const u32x2*>(vp + lane * 8);
  };
  if (np > 0) {
#pragma unroll
    for (int u = 0; u < PPI; ++u) {
      const int64_t row = page_row(u);
      load_k(u, row);
#pragma unroll
      for (int t = 0; t < kPageTokens; ++t) load_v(u, row, t);
    }
  }
  for (int q0 = 0; q0 < np; q0 += PPI) {
    int64_t nrow[PPI];
    f32x4 sc[PPI];
    float skj[PPI][4], svj[PPI][4];
#pragma unroll
    for (int u = 0; u < PPI; ++u) {
      nrow[u] = page_row(q0 + PPI + u);
      sc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (FP8) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_bf16(ka[u][r].x, ka[u][r].y),
                                                          __builtin_bit_cast(bf16x8, qb[2 * r]),
                                                          sc[u], 0, 0, 0);
          sc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_bf16(ka[u][r].z, ka[u][r].w),
                                                          __builtin_bit_cast(bf16x8, qb[2 * r + 1]),
                                                          sc[u], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          skj[u][i] = sk[u][i];
          svj[u][i] = svs[u][i];
        }
      } else {
#pragma unroll
        for (int s = 0; s < 8; ++s)
          sc[u] = mfma16<F16>(ka[u][s], qb[s], sc[u]);
      }
      load_k(u, nrow[u]);
    }

    // online softmax for head n over this iteration's tokens 16u + 4g + i
    float sv[PPI][4], pm = -INFINITY;
#pragma unroll
    for (int u = 0; u < PPI; ++u) {
      const int q = q0 + u;
      const bool ok = q < np && ((badmask >> q) & 1u) == 0;
      const int64_t tok0 = (p0 + (int64_t)kAttnWaves * q) * kPageTokens + 4 * g;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float score = FP8 ? sc[u][i] * skj[u][i] : sc[u][i];
        sv[u][i] = ok && tok0 + i < len ? score * a.scale_log2 : -INFINITY;
        pm = fmaxf(pm, sv[u][i]);
      }
    }
    pm = fmaxf(pm, __shfl_xor(pm, 16));
    pm = fmaxf(pm, __shfl_xor(pm, 32));
    const float m_new = fmaxf(m_run, pm);
    // -inf only while every page so far was masked: exponents then stay -inf
    const float m_ref = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2_fast(m_run - m_ref);
    float ps = 0.f;
#pragma unroll
    for (int u = 0; u < PPI; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pv = exp2_fast(sv[u][i] - m_ref);
        ps += pv;
        p_lds[wave][16 * u + 4 * g + i][n] = FP8 ? pv * svj[u][i] : pv;
      }
    ps += __shfl_xor(ps, 16);
    ps += __shfl_xor(ps, 32);
    l_run = l_run * alpha + ps;
    m_run = m_new;
    if (g == 0) al_lds[wave][n] = alpha;
    wave_sync();
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float al = al_lds[wave][h];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) o[h][jj] *= al;
    }
#pragma unroll
    for (int u = 0; u < PPI; ++u)
#pragma unroll
      for (int t = 0; t < kPageTokens; ++t) {
        float v0, v1, v2, v3;
        if constexpr (FP8) {
          const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)vr[u][t], false);
          const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)vr[u][t], true);
          v0 = lo.x;
          v1 = lo.y;
          v2 = hi.x;
          v3 = hi.y;
        } else if constexpr (F16) {
          v0 = f16_lo(vr[u][t].x);
          v1 = f16_hi(vr[u][t].x);
          v2 = f16_lo(vr[u][t].y);
          v3 = f16_hi(vr[u][t].y);
        } else {
          v0 = bf16_lo(vr[u][t].x);
          v1 = bf16_hi(vr[u][t].x);
          v2 = bf16_lo(vr[u][t].y);
          v3 = bf16_hi(vr[u][t].y);
        }
        load_v(u, nrow[u], t);
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const float pt = p_lds[wave][16 * u + t][h];
          o[h][0] += pt * v0;
          o[h][1] += pt * v1;
          o[h][2] += pt * v2;
          o[h][3] += pt * v3;
        }
      }
    wave_sync();  // the next iteration rewrites this wave's tiles
  }

  // merge the waves' (max, sum, output) per head
  if (g == 0 && n < G) {
    m_w[wave][n] = m_run;
    l_w[wave][n] = l_run;
  }
#pragma unroll
  for (int h = 0; h < G; ++h)
    *reinterpret_cast<f32x4*>(&o_w[wave][h][4 * lane]) = f32x4{o[h][0], o[h][1], o[h][2], o[h][3]};
  __syncthreads();
  const int d = threadIdx.x;  // one dim per thread
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, m_w[w][h]);
    float O = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      const float f = m_w[w][h] == -INFINITY ? 0.f : exp2_fast(m_w[w][h] - M);
      O += f * o_w[w][h][d];
      L += f * l_w[w][h];
    }
    if (nch == 1) {
      reinterpret_cast<uint16_t*>(out + h * kRowBytes)[d] = out_bits<F16>(L > 0.f ? O / L : 0.f);
    } else {
      const int64_t at = ((b * a.hkv + hk) * a.chunks + c) * G + h;
      a.part[at * kHeadDim + d] = O;
      if (d == 0) {
        a.ml[at * 2] = M;
        a.ml[at * 2 + 1] = L;
      }
    }
  }
}

template <int G, bool FP8, bool F16>
// two workgroups per CU: without the bound the G = 8 kernels take 256 VGPRs
// plus accumulation registers, one wave per SIMD
__global__ __launch_bounds__(kAttnThreads, 2) void attn_chunk_kernel(AttnArgs a) {
  static_assert(G >= 1 && G <= 8, "query heads per KV head");
  __shared__ float p_lds[kAttnWaves][kIterTokens][16];  // [wave][token][head] probabilities
  __shared__ float al_lds[kAttnWaves][16];              // [wave][head] rescale factor
  __shared__ float m_w[kAttnWaves][G], l_w[kAttnWaves][G];
  __shared__ __attribute__((aligned(16))) float o_w[kAttnWaves][G][kHeadDim];
  // The work list, the same in every workgroup: first the full 1024-token
  // chunks of all (sequence, KV head) pairs, pair-major, then each pair's
  // last, shorter chunk (or the zeros of an empty pair) with the longest
  // first, so that the short items fill the end of the launch.
  __shared__ int32_t first[kMaxPairs + 1];  // first full-chunk item of each pair
  __shared__ int32_t tail_pair[kMaxPairs];  // pairs with a short chunk, longest first
  __shared__ uint8_t tail_key[kMaxPairs];   // its length class, or kTailNone
  __shared__ int32_t class_at[kTailClasses];         // next free slot of each class
  __shared__ int32_t class_wave[kAttnWaves][kTailClasses];
  __shared__ int32_t wave_tot[kAttnWaves];
  __shared__ int32_t item_sh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid < kTailClasses) class_at[tid] = 0;
  __syncthreads();
  // pass 1, 256 pairs per round: full-chunk counts and their exclusive
  // prefix, the short chunk's class and the class sizes
  int32_t total = 0;
  for (int base = 0; base < a.pairs; base += kAttnThreads) {
    const int pr = base + tid;
    int32_t cnt = 0;
    if (pr < a.pairs) {
      const int64_t len = attn_len(a, pr / a.hkv, blockIdx.x == 0 && pr % a.hkv == 0);
      cnt = (int32_t)(len / kChunk);
      const int32_t rem = (int32_t)(len % kChunk);
      const bool tail = rem != 0 || len == 0;  // an empty pair still zeroes its output
      const int key = tail ? kTailClasses - 1 - rem / (kChunk / kTailClasses) : kTailNone;
      tail_key[pr] = (uint8_t)key;
      if (tail) atomicAdd(&class_at[key], 1);
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
    if (pr < a.pairs) first[pr] = at;
    total += round;
    __syncthreads();  // wave_tot is rewritten by the next round
  }
  const int32_t total_full = total;
  // class sizes -> their first slots (exclusive scan of 32 counts in wave 0)
  if (wave == 0) {
    const int32_t n_c = lane < kTailClasses ? class_at[lane] : 0;
    int32_t incl = n_c;
#pragma unroll
    for (int dd = 1; dd < 64; dd <<= 1) {
      const int32_t o = __shfl_up(incl, dd);
      if (lane >= dd) incl += o;
    }
    if (lane < kTailClasses) class_at[lane] = incl - n_c;
    if (lane == 63) item_sh = incl;  // number of short chunks
  }
  __syncthreads();
  const int32_t n_tail = __builtin_amdgcn_readfirstlane(item_sh);
  // pass 2: each short chunk's slot, stable by pair index within its class
  for (int base = 0; base < a.pairs; base += kAttnThreads) {
    const int pr = base + tid;
    const int key = pr < a.pairs ? tail_key[pr] : kTailNone;
    int my_rank = 0;
    for (int c = 0; c < kTailClasses; ++c) {
      const uint64_t m = __ballot(key == c);
      if (key == c) my_rank = __popcll(m & ((1ull << lane) - 1));
      if (lane == 0) class_wave[wave][c] = __popcll(m);
    }
    __syncthreads();
    if (key != kTailNone) {
      int32_t slot = class_at[key] + my_rank;
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) slot += w < wave ? class_wave[w][key] : 0;
      tail_pair[slot] = pr;
    }
    __syncthreads();  // class_at and class_wave are updated below / rewritten next round
    if (tid < kTailClasses) {
      int32_t add = 0;
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) add += class_wave[w][tid];
      class_at[tid] += add;
    }
    __syncthreads();
  }
  if (tid == 0) first[a.pairs] = total_full;
  // The first round is static: workgroup w takes item w. Later items come from
  // the counter, offset by the grid, and only when there are more items than
  // workgroups. A launch of 1024 workgroups all hitting one device-scope
  // atomic at their start, and again at their exit, cost 4-12 us per launch
  // (3-16 %) on short contexts.
  const int32_t n_items = total_full + n_tail;
  for (int32_t round = 0;; ++round) {
    __syncthreads();  // the lists written; the previous item's LDS reads done
    if (round > 0) {
      if (n_items <= (int32_t)gridDim.x) break;  // uniform
      if (tid == 0) item_sh = (int32_t)gridDim.x + atomicAdd(a.queue, 1);
    } else if (tid == 0) {
      item_sh = (int32_t)blockIdx.x;
    }
    __syncthreads();
    // work-item values are uniform: scalar registers (readfirstlane)
    const int32_t item = __builtin_amdgcn_readfirstlane(item_sh);
    if (item >= n_items || item < 0) break;  // uniform: every workgroup ends here
    int32_t pair, c;
    if (item < total_full) {  // the last pair whose full chunks start at or before `item`
      int lo = 0, hi = a.pairs - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (first[mid] <= item) lo = mid; else hi = mid - 1;
      }
      pair = lo;
      c = item - first[lo];
    } else {
      pair = tail_pair[item - total_full];
      c = -1;  // the pair's last chunk, index len / kChunk
    }
    pair = __builtin_amdgcn_readfirstlane(pair);
    c = __builtin_amdgcn_readfirstlane(c);
    const int64_t b = pair / a.hkv, hk = pair % a.hkv;
    const int64_t len = attn_len(a, b, false);
    if (c < 0) c = (int32_t)(len / kChunk);
    attn_chunk<G, FP8, F16>(a, b, hk, c, len, (len + kChunk - 1) / kChunk, p_lds, al_lds, m_w, l_w,
                       o_w);
  }
}

// Merges the chunk states of one (sequence, KV head, query head) of a
// sequence longer than one chunk: the chunks' maximum by a block reduction,
// then a thread per dim sums the rescaled partial rows (loads 8 chunks deep).
template <int G, bool F16>
__global__ __launch_bounds__(kAttnThreads) void attn_merge_kernel(AttnArgs a) {
  __shared__ float red[kAttnWaves];
  // the chunk kernel has finished (stream order): its counter starts from
  // zero for the next call
  if (blockIdx.x == 0 && threadIdx.x == 0) a.queue[0] = 0;
  const int64_t pr = blockIdx.x / G;
  const int h = blockIdx.x % G;
  const int64_t b = pr / a.hkv;
  const int64_t len = attn_len(a, b, false);
  const int64_t nch = (len + kChunk - 1) / kChunk;
  if (nch <= 1) return;  // written by the chunk kernel
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t at0 = pr * a.chunks * G + h;  // chunk c: at0 + c * G
  float M = -INFINITY;
  for (int64_t c = tid; c < nch; c += kAttnThreads) M = fmaxf(M, a.ml[(at0 + c * G) * 2]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
  if (lane == 0) red[wave] = M;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, red[w]);
  float O = 0.f, L = 0.f;
#pragma unroll 8
  for (int64_t c = 0; c < nch; ++c) {
    const int64_t at = at0 + c * G;
    const float m = ld_const(a.ml + at * 2);
    const float f = m == -INFINITY ? 0.f : exp2_fast(m - M);
    O += f * a.part[at * kHeadDim + tid];
    L += f * ld_const(a.ml + at * 2 + 1);
  }
  uint8_t* out = a.out + (pr * G + h) * kRowBytes;
  reinterpret_cast<uint16_t*>(out)[tid] = out_bits<F16>(L > 0.f ? O / L : 0.f);
}

inline int64_t attn_chunks(int32_t max_seq_len) {
  return ((int64_t)max_seq_len + kChunk - 1) / kChunk;
}

// Workgroups of the chunk kernel: as many as are resident at once (CUs x the
// kernel's occupancy, 2 per CU for four query heads), so that every
// workgroup's static first item starts at once and the counter hands out the
// rest in list order. A grid of 4 per CU left the second half's first items,
// full chunks, to the end of the launch: 304.7 against 295.4 us per bf16
// launch at batch 256, 102.4 against 100.4 us in the serving workload.
template <int G, bool FP8, bool F16>
int attn_grid() {
  static int grid[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 512;
  if (grid[dev] == 0) {
    int n = 0, per = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, attn_chunk_kernel<G, FP8, F16>,
                                                     kAttnThreads, 0) != hipSuccess || per <= 0)
      per = 2;
    grid[dev] = n * per;
  }
  return grid[dev];
}

template <int G, bool FP8, bool F16>
void launch_attn(const AttnArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((attn_chunk_kernel<G, FP8, F16>), dim3((unsigned)attn_grid<G, FP8, F16>()),
                     dim3(kAttnThreads), 0, st, a);
  // the merge kernel also resets the work counter: one workgroup when no
  // sequence spans two chunks
  hipLaunchKernelGGL((attn_merge_kernel<G, F16>), dim3(a.chunks > 1 ? (unsigned)(a.pairs * G) : 1u),
                     dim3(kAttnThreads), 0, st, a);
}

}  // namespace
}  // namespace mkv

using namespace mkv;

constexpr int64_t kQueueBytes = 256;  // the work counters, at the workspace's start

extern "C" int64_t mkv_decode_attention_workspace_bytes(int32_t batch, int32_t num_kv_heads,
                                                        int32_t num_q_heads, int32_t max_seq_len) {
  if (batch < 0 || num_kv_heads <= 0 || num_q_heads <= 0 || max_seq_len < 0) return -1;
  const int64_t chunks = attn_chunks(max_seq_len);
  return kQueueBytes + (chunks <= 1 ? 0 : (int64_t)batch * num_q_heads * chunks * (kHeadDim + 2) * 4);
}

namespace {

// Element kinds of the pool the entry points read.
enum AttnKind { kAttnBf16, kAttnFp8, kAttnF16 };

template <int G>
void launch_kind(AttnKind kind, const AttnArgs& a, hipStream_t st) {
  if (kind == kAttnFp8)
    launch_attn<G, true, false>(a, st);
  else if (kind == kAttnF16)
    launch_attn<G, false, true>(a, st);
  else
    launch_attn<G, false, false>(a, st);
}

// Shared by the entry points: `fn` names the caller in error messages; the
// scale planes are null for 16-bit caches.
int decode_attention(const char* fn, AttnKind kind, const void* q, const void* k_cache,
                     const void* v_cache, const float* k_scales, const float* v_scales,
                     int64_t num_pages, int32_t num_kv_heads, int32_t num_q_heads,
                     int32_t head_dim, const int32_t* page_table, int64_t table_stride,
                     int32_t table_width, const int32_t* seq_lens, int32_t batch,
                     int32_t max_seq_len, float softmax_scale, void* out, void* workspace,
                     int64_t workspace_bytes, int32_t* err, void* stream) {
  clear_error();
  MKV_REQUIRE(batch >= 0 && num_pages > 0 && num_kv_heads > 0 && num_q_heads > 0 &&
                  table_width >= 0 && table_stride >= table_width && max_seq_len >= 0,
              MKV_E_INVALID, "%s: bad sizes", fn);
  MKV_REQUIRE(head_dim == kHeadDim, MKV_E_UNSUPPORTED, "%s: head_dim %d unsupported (256)", fn,
              head_dim);
  const int32_t G = num_q_heads / num_kv_heads;
  MKV_REQUIRE(G * num_kv_heads == num_q_heads && (G == 1 || G == 2 || G == 4 || G == 8),
              MKV_E_UNSUPPORTED, "%s: %d query heads per KV head unsupported (1, 2, 4, 8)", fn,
              num_q_heads / num_kv_heads);
  if (batch == 0) return MKV_OK;
  MKV_REQUIRE(q && k_cache && v_cache && page_table && seq_lens && out && err &&
                  (kind != kAttnFp8 || (k_scales && v_scales)),
              MKV_E_INVALID, "%s: null pointer", fn);
  MKV_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out),
              MKV_E_ALIGN, "%s: q, caches and out must be 16-byte aligned", fn);
  MKV_REQUIRE(kind != kAttnFp8 || (aligned4(k_scales) && aligned4(v_scales)), MKV_E_ALIGN,
              "%s: scale planes must be 4-byte aligned", fn);
  MKV_REQUIRE((int64_t)batch * num_kv_heads <= kMaxPairs, MKV_E_UNSUPPORTED,
              "%s: batch x KV heads above %d", fn, kMaxPairs);
  MKV_REQUIRE(max_seq_len <= (1 << 24), MKV_E_UNSUPPORTED, "%s: max_seq_len above 2^24", fn);
  const int64_t need = mkv_decode_attention_workspace_bytes(batch, num_kv_heads, num_q_heads,
                                                            max_seq_len);
  MKV_REQUIRE(workspace && workspace_bytes >= need && aligned16(workspace), MKV_E_INVALID,
              "%s: workspace of %lld bytes (16-byte aligned) required", fn, (long long)need);
  AttnArgs a;
  a.q = static_cast<const uint8_t*>(q);
  a.k = static_cast<const uint8_t*>(k_cache);
  a.v = static_cast<const uint8_t*>(v_cache);
  a.ks = k_scales;
  a.vs = v_scales;
  a.table = page_table;
  a.lens = seq_lens;
  a.out = static_cast<uint8_t*>(out);
  const int64_t chunks = attn_chunks(max_seq_len);
  const int64_t part_floats = (int64_t)batch * num_q_heads * chunks * kHeadDim;
  a.queue = static_cast<int32_t*>(workspace);
  a.part = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kQueueBytes);
  a.ml = a.part + part_floats;
  a.num_pages = num_pages;
  a.tstride = table_stride;
  a.twidth = table_width;
  a.hkv = num_kv_heads;
  a.chunks = (int32_t)chunks;
  a.max_len = max_seq_len;
  a.pairs = (int32_t)((int64_t)batch * num_kv_heads);
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.err = err;
  const hipStream_t st = as_stream(stream);
  switch (G) {
    case 1: launch_kind<1>(kind, a, st); break;
    case 2: launch_kind<2>(kind, a, st); break;
    case 4: launch_kind<4>(kind, a, st); break;
    default: launch_kind<8>(kind, a, st); break;
  }
  return check_launch(fn);
}

}  // namespace

extern "C" int mkv_decode_attention_bf16(const void* q, const void* k_cache, const void* v_cache,
                                         int64_t num_pages, int32_t num_kv_heads,
                                         int32_t num_q_heads, int32_t head_dim,
                                         const int32_t* page_table, int64_t table_stride,
                                         int32_t table_width, const int32_t* seq_lens,
                                         int32_t batch, int32_t max_seq_len, float softmax_scale,
                                         void* out, void* workspace, int64_t workspace_bytes,
                                         int32_t* err, void* stream) {
  return decode_attention("mkv_decode_attention_bf16", kAttnBf16, q, k_cache, v_cache, nullptr,
                          nullptr, num_pages, num_kv_heads, num_q_heads, head_dim, page_table,
                          table_stride, table_width, seq_lens, batch, max_seq_len, softmax_scale,
                          out, workspace, workspace_bytes, err, stream);
}

extern "C" int mkv_decode_attention_fp8(const void* q, const void* k_codes, const void* v_codes,
                                        const float* k_scales, const float* v_scales,
                                        int64_t num_pages, int32_t num_kv_heads,
                                        int32_t num_q_heads, int32_t head_dim,
                                        const int32_t* page_table, int64_t table_stride,
                                        int32_t table_width, const int32_t* seq_lens,
                                        int32_t batch, int32_t max_seq_len, float softmax_scale,
                                        void* out, void* workspace, int64_t workspace_bytes,
                                        int32_t* err, void* stream) {
  return decode_attention("mkv_decode_attention_fp8", kAttnFp8, q, k_codes, v_codes, k_scales,
                          v_scales, num_pages, num_kv_heads, num_q_heads, head_dim, page_table,
                          table_stride, table_width, seq_lens, batch, max_seq_len, softmax_scale,
                          out, workspace, workspace_bytes, err, stream);
}

extern "C" int mkv_decode_attention_f16(const void* q, const void* k_cache, const void* v_cache,
                                        int64_t num_pages, int32_t num_kv_heads,
                                        int32_t num_q_heads, int32_t head_dim,
                                        const int32_t* page_table, int64_t table_stride,
                                        int32_t table_width, const int32_t* seq_lens,
                                        int32_t batch, int32_t max_seq_len, float softmax_scale,
                                        void* out, void* workspace, int64_t workspace_bytes,
                                        int32_t* err, void* stream) {
  return decode_attention("mkv_decode_attention_f16", kAttnF16, q, k_cache, v_cache, nullptr,
                          nullptr, num_pages, num_kv_heads, num_q_heads, head_dim, page_table,
                          table_stride, table_width, seq_lens, batch, max_seq_len, softmax_scale,
                          out, workspace, workspace_bytes, err, stream);
}

// ---------------------------------------------------------------------------
// The same bf16 decode attention for callers that cannot allocate (code under
// HIP graph capture, tight serving loops): the workspace is a file-scope
// device array, one copy per GPU, held until the process ends.
// ---------------------------------------------------------------------------
namespace {

// Room for the work counters and the chunk partials of batch x query heads x
// chunks <= 48,770 (e.g. batch 256, 4 query heads, max_seq_len up to 47 x
// 1024 tokens).
constexpr int64_t kNoAllocScratchBytes = 48ll << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

__global__ void zero_queue_kernel(int32_t* queue) {
  if (threadIdx.x < kQueueBytes / 4) queue[threadIdx.x] = 0;
}

// The current device's copy of `scratch`. In host code the array's name is
// only a stand-in for the symbol: its device address comes from
// hipGetSymbolAddress, once per device (with that device current), and only
// that address is ever handed to a kernel. The first call on a device also
// zeroes the work counters on the caller's stream (a fill kernel, not a
// memset node); every call leaves them zero again (the merge kernel resets
// them), as it does for a caller's workspace.
int scratch_of_current_device(const char* fn, hipStream_t st, void** out) {
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
    hipLaunchKernelGGL(zero_queue_kernel, dim3(1), dim3(64), 0, st, static_cast<int32_t*>(p));
    const int rc = check_launch(fn);
    if (rc != MKV_OK) return rc;
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
  const int64_t need =
      mkv_decode_attention_workspace_bytes(batch, num_kv_heads, num_q_heads, max_seq_len);
  MKV_REQUIRE(need <= kNoAllocScratchBytes, MKV_E_UNSUPPORTED,
              "%s: batch %d x %d query heads x %lld chunks of 1024 tokens need %lld bytes of "
              "scratch, the static scratch holds %lld",
              fn, batch, num_q_heads, (long long)attn_chunks(max_seq_len), (long long)need,
              (long long)kNoAllocScratchBytes);
  if (batch == 0) return decode_attention(fn, kAttnBf16, q, k_cache, v_cache, nullptr, nullptr,
                                          num_pages, num_kv_heads, num_q_heads, head_dim,
                                          page_table, table_stride, table_width, seq_lens, batch,
                                          max_seq_len, softmax_scale, out, nullptr, 0, err,
                                          stream);
  void* ws = nullptr;
  const int rc = scratch_of_current_device(fn, as_stream(stream), &ws);
  if (rc != MKV_OK) return rc;
  return decode_attention(fn, kAttnBf16, q, k_cache, v_cache, nullptr, nullptr, num_pages,
                          num_kv_heads, num_q_heads, head_dim, page_table, table_stride,
                          table_width, seq_lens, batch, max_seq_len, softmax_scale, out, ws,
                          kNoAllocScratchBytes, err, stream);
}
