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
// A workgroup (4 waves) takes a 512-token chunk of one sequence and KV head;
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
//     output) per chunk to the caller's workspace and a second kernel merges.
#include <math.h>

#include "mkv_device.h"

namespace mkv {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kHeadDim = 256;
constexpr int kRowBytes = kHeadDim * 2;  // one bf16 K or V row of one KV head
constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr int kPageTokens = 16;
constexpr int kChunk = 512;  // tokens per workgroup
constexpr int kChunkPages = kChunk / kPageTokens;

struct AttnArgs {
  const uint8_t* q;  // [B, Hkv * G, 256] bf16
  const uint8_t* k;  // [P, 16, Hkv, 256] bf16
  const uint8_t* v;
  const int32_t* table;  // [B, tstride] int32
  const int32_t* lens;   // [B] int32
  uint8_t* out;          // [B, Hkv * G, 256] bf16
  float* part;           // [B, Hkv, chunks, G, 256] unnormalised chunk outputs
  float* ml;             // [B, Hkv, chunks, G, 2] chunk (max, sum), log2 units
  int64_t num_pages, tstride;
  int32_t twidth, hkv, chunks, max_len;
  float scale_log2;  // softmax_scale * log2(e)
  int32_t* err;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return bits_f32(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return bits_f32(w & 0xffff0000u); }
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

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

template <int G>
__global__ __launch_bounds__(kAttnThreads) void attn_chunk_kernel(AttnArgs a) {
  static_assert(G >= 1 && G <= 8, "query heads per KV head");
  __shared__ float p_lds[kAttnWaves][kPageTokens][16];  // [wave][token][head] probabilities
  __shared__ float al_lds[kAttnWaves][16];              // [wave][head] rescale factor
  __shared__ float m_w[kAttnWaves][G], l_w[kAttnWaves][G];
  __shared__ __attribute__((aligned(16))) float o_w[kAttnWaves][G][kHeadDim];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int64_t b = blockIdx.y / a.hkv, hk = blockIdx.y % a.hkv;
  const int c = blockIdx.x;
  const int64_t len = attn_len(a, b, c == 0 && threadIdx.x == 0);
  const int64_t nch = (len + kChunk - 1) / kChunk;
  uint8_t* out = a.out + (b * a.hkv + hk) * G * kRowBytes;
  if (len == 0) {  // nothing to attend to: zeros
    if (c == 0)
      for (int i = threadIdx.x; i < G * kRowBytes / 16; i += kAttnThreads)
        st16(out + i * 16, u32x4{0u, 0u, 0u, 0u});
    return;
  }
  if (c >= nch) return;

  // the G query heads as the B operand, in the K rows' chunk order
  bf16x8 qb[8];
  const uint8_t* qrow = a.q + ((b * a.hkv + hk) * G + (n < G ? n : 0)) * kRowBytes;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const u32x4 w = n < G ? ld16(qrow + (4 * s + g) * 16) : u32x4{0u, 0u, 0u, 0u};
    qb[s] = __builtin_bit_cast(bf16x8, w);
  }
  float m_run = -INFINITY, l_run = 0.f;  // head n
  float o[G][4];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int j = 0; j < 4; ++j) o[h][j] = 0.f;

  const int64_t tok_stride = (int64_t)a.hkv * kRowBytes;
  const int64_t pages = (len + kPageTokens - 1) / kPageTokens;
  const int64_t p_end = (c + 1) * (int64_t)kChunkPages < pages ? (c + 1) * (int64_t)kChunkPages : pages;
  const int32_t* trow = a.table + b * a.tstride;
  for (int64_t p = c * (int64_t)kChunkPages + wave; p < p_end; p += kAttnWaves) {
    const int32_t pid = ld_const(trow + p);
    if (pid < 0 || pid >= a.num_pages) {  // wave-uniform: the page is skipped
      if (lane == 0) raise_err(a.err, MKV_DEVERR_PAGE);
      continue;
    }
    const int64_t base = ((int64_t)pid * kPageTokens * a.hkv + hk) * kRowBytes;
    const uint8_t* kp = a.k + base + n * tok_stride;
    const uint8_t* vp = a.v + base + lane * 8;
    bf16x8 ka[8];
    u32x2 vr[kPageTokens];
#pragma unroll
    for (int s = 0; s < 8; ++s) ka[s] = __builtin_bit_cast(bf16x8, ld16(kp + (4 * s + g) * 16));
#pragma unroll
    for (int t = 0; t < kPageTokens; ++t)
      vr[t] = *reinterpret_cast<const u32x2*>(vp + t * tok_stride);
    f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s) sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[s], qb[s], sc, 0, 0, 0);

    // online softmax for head n over this page's tokens 4g .. 4g+3
    const int64_t tok0 = p * kPageTokens + 4 * g;
    float sv[4], pm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sv[i] = tok0 + i < len ? sc[i] * a.scale_log2 : -INFINITY;
      pm = fmaxf(pm, sv[i]);
    }
    pm = fmaxf(pm, __shfl_xor(pm, 16));
    pm = fmaxf(pm, __shfl_xor(pm, 32));
    const float m_new = fmaxf(m_run, pm);  // finite: a page holds at least one valid token
    const float alpha = exp2_fast(m_run - m_new);
    float pv[4], ps = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pv[i] = exp2_fast(sv[i] - m_new);
      ps += pv[i];
    }
    ps += __shfl_xor(ps, 16);
    ps += __shfl_xor(ps, 32);
    l_run = l_run * alpha + ps;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < 4; ++i) p_lds[wave][4 * g + i][n] = pv[i];
    if (g == 0) al_lds[wave][n] = alpha;
    wave_sync();
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float al = al_lds[wave][h];
#pragma unroll
      for (int j = 0; j < 4; ++j) o[h][j] *= al;
    }
#pragma unroll
    for (int t = 0; t < kPageTokens; ++t) {
      const float v0 = bf16_lo(vr[t].x), v1 = bf16_hi(vr[t].x);
      const float v2 = bf16_lo(vr[t].y), v3 = bf16_hi(vr[t].y);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float pt = p_lds[wave][t][h];
        o[h][0] += pt * v0;
        o[h][1] += pt * v1;
        o[h][2] += pt * v2;
        o[h][3] += pt * v3;
      }
    }
    wave_sync();  // the next page rewrites this wave's tiles
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
      reinterpret_cast<uint16_t*>(out + h * kRowBytes)[d] = f32_to_bf16_rne(L > 0.f ? O / L : 0.f);
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

// Merges the chunk states of sequences longer than one chunk.
template <int G>
__global__ __launch_bounds__(kAttnThreads) void attn_merge_kernel(AttnArgs a) {
  const int64_t b = blockIdx.x / a.hkv, hk = blockIdx.x % a.hkv;
  const int64_t len = attn_len(a, b, false);
  const int64_t nch = (len + kChunk - 1) / kChunk;
  if (nch <= 1) return;  // written by the chunk kernel
  const int d = threadIdx.x;
  uint8_t* out = a.out + (b * a.hkv + hk) * G * kRowBytes;
  const int64_t at0 = (b * a.hkv + hk) * a.chunks * G;
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float M = -INFINITY;
    for (int64_t c = 0; c < nch; ++c) M = fmaxf(M, a.ml[(at0 + c * G + h) * 2]);
    float O = 0.f, L = 0.f;
    for (int64_t c = 0; c < nch; ++c) {
      const int64_t at = at0 + c * G + h;
      const float m = a.ml[at * 2];
      const float f = m == -INFINITY ? 0.f : exp2_fast(m - M);
      O += f * a.part[at * kHeadDim + d];
      L += f * a.ml[at * 2 + 1];
    }
    reinterpret_cast<uint16_t*>(out + h * kRowBytes)[d] = f32_to_bf16_rne(L > 0.f ? O / L : 0.f);
  }
}

inline int64_t attn_chunks(int32_t max_seq_len) {
  return ((int64_t)max_seq_len + kChunk - 1) / kChunk;
}

template <int G>
void launch_attn(const AttnArgs& a, int64_t bh, hipStream_t st) {
  hipLaunchKernelGGL(attn_chunk_kernel<G>, dim3((unsigned)(a.chunks > 0 ? a.chunks : 1), (unsigned)bh),
                     dim3(kAttnThreads), 0, st, a);
  if (a.chunks > 1)
    hipLaunchKernelGGL(attn_merge_kernel<G>, dim3((unsigned)bh), dim3(kAttnThreads), 0, st, a);
}

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int64_t mkv_decode_attention_workspace_bytes(int32_t batch, int32_t num_kv_heads,
                                                        int32_t num_q_heads, int32_t max_seq_len) {
  if (batch < 0 || num_kv_heads <= 0 || num_q_heads <= 0 || max_seq_len < 0) return -1;
  const int64_t chunks = attn_chunks(max_seq_len);
  if (chunks <= 1) return 0;
  return (int64_t)batch * num_q_heads * chunks * (kHeadDim + 2) * 4;
}

extern "C" int mkv_decode_attention_bf16(const void* q, const void* k_cache, const void* v_cache,
                                         int64_t num_pages, int32_t num_kv_heads,
                                         int32_t num_q_heads, int32_t head_dim,
                                         const int32_t* page_table, int64_t table_stride,
                                         int32_t table_width, const int32_t* seq_lens,
                                         int32_t batch, int32_t max_seq_len, float softmax_scale,
                                         void* out, void* workspace, int64_t workspace_bytes,
                                         int32_t* err, void* stream) {
  clear_error();
  MKV_REQUIRE(batch >= 0 && num_pages > 0 && num_kv_heads > 0 && num_q_heads > 0 &&
                  table_width >= 0 && table_stride >= table_width && max_seq_len >= 0,
              MKV_E_INVALID, "mkv_decode_attention_bf16: bad sizes");
  MKV_REQUIRE(head_dim == kHeadDim, MKV_E_UNSUPPORTED,
              "mkv_decode_attention_bf16: head_dim %d unsupported (256)", head_dim);
  const int32_t G = num_q_heads / num_kv_heads;
  MKV_REQUIRE(G * num_kv_heads == num_q_heads && (G == 1 || G == 2 || G == 4 || G == 8),
              MKV_E_UNSUPPORTED,
              "mkv_decode_attention_bf16: %d query heads per KV head unsupported (1, 2, 4, 8)",
              num_q_heads / num_kv_heads);
  if (batch == 0) return MKV_OK;
  MKV_REQUIRE(q && k_cache && v_cache && page_table && seq_lens && out && err, MKV_E_INVALID,
              "mkv_decode_attention_bf16: null pointer");
  MKV_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out),
              MKV_E_ALIGN, "mkv_decode_attention_bf16: q, caches and out must be 16-byte aligned");
  MKV_REQUIRE((int64_t)batch * num_kv_heads <= 65535, MKV_E_UNSUPPORTED,
              "mkv_decode_attention_bf16: batch x KV heads above 65535");
  const int64_t need = mkv_decode_attention_workspace_bytes(batch, num_kv_heads, num_q_heads,
                                                            max_seq_len);
  MKV_REQUIRE(need == 0 || (workspace && workspace_bytes >= need && aligned16(workspace)),
              MKV_E_INVALID,
              "mkv_decode_attention_bf16: workspace of %lld bytes (16-byte aligned) required",
              (long long)need);
  AttnArgs a;
  a.q = static_cast<const uint8_t*>(q);
  a.k = static_cast<const uint8_t*>(k_cache);
  a.v = static_cast<const uint8_t*>(v_cache);
  a.table = page_table;
  a.lens = seq_lens;
  a.out = static_cast<uint8_t*>(out);
  const int64_t chunks = attn_chunks(max_seq_len);
  const int64_t part_floats = (int64_t)batch * num_q_heads * chunks * kHeadDim;
  a.part = static_cast<float*>(workspace);
  a.ml = need ? a.part + part_floats : nullptr;
  a.num_pages = num_pages;
  a.tstride = table_stride;
  a.twidth = table_width;
  a.hkv = num_kv_heads;
  a.chunks = (int32_t)chunks;
  a.max_len = max_seq_len;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.err = err;
  const int64_t bh = (int64_t)batch * num_kv_heads;
  const hipStream_t st = as_stream(stream);
  switch (G) {
    case 1: launch_attn<1>(a, bh, st); break;
    case 2: launch_attn<2>(a, bh, st); break;
    case 4: launch_attn<4>(a, bh, st); break;
    default: launch_attn<8>(a, bh, st); break;
  }
  return check_launch("mkv_decode_attention_bf16");
}
