// mkv_prefill.hip — varlen prefill attention (gfx950, MFMA): the math of
// attn_prefill (muserve/kernels/attention.py:6-25, flash_attn_varlen_func)
// over contiguous K/V, and the same over the paged pool for chunked prefill
// (a chunk's queries attend to the sequence's cached prefix and to
// themselves).
//
// Sequence b has nq queries and nk keys; query t sits at position nk - nq + t
// (causal masking aligned to the bottom-right corner) and, when causal,
// attends to positions 0 .. nk - nq + t. Query head h reads KV head h / 4.
//
// A workgroup (8 waves) takes 32 query tokens of one sequence and KV head;
// wave w holds query head 4*hk + w % 4 for tokens 16 (w / 4) .. +15, so the 8
// waves share every K/V tile through LDS. K/V tiles are double-buffered in
// LDS with one barrier per tile: while tile i is computed, tile i + 1 goes
// from registers into the other buffer and tile i + 2's global loads are
// issued. Per 64-token KV tile:
//   * the tile is staged in LDS, K and V both as token rows (16-byte
//     stores); the S product reads K operands as 16-byte LDS loads, the P V
//     product reads V operands with gfx950's transposing LDS load
//     (ds_read_b64_tr_b16), so V is never transposed by hand;
//   * S = Q K^T on MFMA (v_mfma_f32_16x16x32_bf16): A = 16 query rows x 32
//     dims held in registers for the whole loop, B = 16 K rows; 8 steps over
//     head_dim 256 for each 16-token quarter;
//   * online softmax in fp32 on the 4 rows x 4 tokens a lane holds (exp2,
//     log2(e) folded into the scale), reductions over the 16 lanes of a row
//     by DPP moves;
//   * P goes through a per-wave LDS tile to become the A operand: a lane
//     rounds its 4 rows of one token to bf16 by packed conversions and stores
//     them as one 8-byte piece of the token-major tile, read back by the same
//     transposing load as V; O += P V on MFMA, 16 blocks of 16 dims.
// The output is O / l, rounded to bf16 once.
#include <math.h>

#include "mkv_device.h"

namespace mkv {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// ds_read_b64_tr_b16: within each group of 16 lanes, lane j names an 8-byte
// row R_j of 4 bf16; lane i receives R_{4e + i/4}[i % 4] as element e (a
// layout probed on the device). Lane j of the group naming
// V[t0 + j/4][d0 + 4 (j % 4) ..] therefore hands lane i the 4 values
// V[t0 .. t0+3][d0 + i]: a column of 4 tokens, the MFMA B-operand order.
__device__ __forceinline__ s16x4 lds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}

constexpr int kPD = 256;           // head_dim
constexpr int kPRow = kPD * 2;     // bytes of one bf16 row
constexpr int kPThreads = 512;     // 8 waves
constexpr int kPWaves = kPThreads / 64;
constexpr int kPG = 4;             // query heads per KV head
constexpr int kQTok = 32;          // query tokens per workgroup (16 per wave)
constexpr int kKvTile = 64;        // KV tokens per step
constexpr int kNQ = kKvTile / 16;  // 16-token quarters of a KV tile
// bf16 per staged K row, padded against bank conflicts of the score operand
// reads: a 16-byte read per lane of rows 16 q + n. Measured on MI355X: a row
// stride of 132 or 140 dwords (+8 or +24 bf16) left 34 % of the LDS's active
// cycles in bank-conflict stalls, 136 dwords (+16) 12 %, and the kernel ran
// 10 % faster.
constexpr int kKStride = kPD + 16;
constexpr int kVStride = kPD + 16;  // bf16 per staged V row
constexpr int kStage = kKvTile * kPRow / 16 / kPThreads;  // 16-byte K (and V) chunks per thread

struct PrefillArgs {
  const uint8_t* q;      // [Tq, Hq, 256] bf16
  const uint8_t* k;      // paged [P, 16, Hkv, 256] or contiguous [Tk, Hkv, 256] bf16
  const uint8_t* v;
  const int32_t* table;  // paged: [B, tstride] page ids; null: contiguous
  int64_t tstride;
  int32_t twidth;
  int64_t kv_units;      // pages (paged) or token rows (contiguous)
  const int32_t* cu_q;   // [B + 1]
  const int32_t* cu_k;   // contiguous: [B + 1]
  const int32_t* lens_k; // paged: [B]
  int64_t num_q;         // query rows Tq
  int32_t max_q;         // the launch's bound on a sequence's queries
  uint8_t* out;          // [Tq, Hq, 256] bf16
  int32_t hkv;
  int32_t causal;
  int32_t splits;        // key ranges per (query tile, KV head); 1: output directly
  int32_t split_len;     // keys per range (a multiple of the KV tile)
  float* part;           // splits > 1: [Tq, Hq, splits, 256] unnormalised outputs
  float* ml;             // splits > 1: [Tq, Hq, splits, 2] (max, sum), log2 units
  float scale_log2;
  int32_t* err;
};

__device__ __forceinline__ uint16_t bf16_bits(float x) { return f32_to_bf16_rne(x); }

// two floats to bf16 (round to nearest even) by one v_cvt_pk_bf16_f32; the
// probabilities it rounds are finite and non-negative
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16_pack(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

// All-reduce over the 16 lanes of a row with DPP moves (VALU, no LDS round
// trip): swap neighbours, swap pairs, mirror within 8, mirror within 16.
// Every lane has a source under these patterns, so the move needs no "old"
// value (bound_ctrl): no zeroing move per step, and the sums fuse into
// v_add_f32_dpp (1.4 % faster than with old = 0).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL,
                                                            0xf, 0xf, true));
}
constexpr int kQuadSwap1 = 0xB1;   // quad_perm [1, 0, 3, 2]
constexpr int kQuadSwap2 = 0x4E;   // quad_perm [2, 3, 0, 1]
constexpr int kHalfMirror = 0x141; // row_half_mirror
constexpr int kMirror = 0x140;     // row_mirror
__device__ __forceinline__ float row_max16(float x) {
  x = fmaxf(x, dpp<kQuadSwap1>(x));
  x = fmaxf(x, dpp<kQuadSwap2>(x));
  x = fmaxf(x, dpp<kHalfMirror>(x));
  return fmaxf(x, dpp<kMirror>(x));
}
__device__ __forceinline__ float row_sum16(float x) {
  x += dpp<kQuadSwap1>(x);
  x += dpp<kQuadSwap2>(x);
  x += dpp<kHalfMirror>(x);
  return x + dpp<kMirror>(x);
}

__global__ __launch_bounds__(kPThreads) void prefill_attn_kernel(PrefillArgs a) {
  // two K/V tile buffers: tile i + 1 is stored while tile i is computed
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][kKvTile][kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][kKvTile][kVStride];
  // P of each wave, token-major: [token][row]
  __shared__ __attribute__((aligned(16))) uint16_t p_lds[kPWaves][kKvTile][16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int64_t b = blockIdx.y, hk = blockIdx.z / a.splits, split = blockIdx.z % a.splits;
  const int32_t qs = a.cu_q[b];
  const int32_t nq_raw = a.cu_q[b + 1] - qs;
  // query offsets outside the buffer, or more queries than the launch covers:
  // flagged; nothing of the sequence (or nothing past the bound) is touched
  const bool q_ok = qs >= 0 && nq_raw >= 0 && (int64_t)qs + nq_raw <= a.num_q;
  if ((!q_ok || nq_raw > a.max_q) && tid == 0 && blockIdx.x == 0 && blockIdx.z == 0)
    raise_err(a.err, MKV_DEVERR_TABLE);
  const int32_t nq = q_ok ? (nq_raw < a.max_q ? nq_raw : a.max_q) : 0;
  const int32_t qt = (int32_t)blockIdx.x * kQTok;  // the workgroup's first query
  if (qt >= nq) return;  // uniform
  const int64_t hq = (int64_t)a.hkv * kPG;
  const int64_t h = hk * kPG + (wave & 3);  // this wave's query head
  const int32_t q0 = qt + 16 * (wave >> 2);  // this wave's first query

  // the sequence's keys: a length checked against what the table (or the
  // buffer) holds; a bad one is flagged and clamped
  int64_t nk, kbase = 0;
  bool bad = false;
  if (a.table) {
    nk = a.lens_k[b];
    const int64_t cap = (int64_t)a.twidth * 16;
    if (nk < 0 || nk > cap) {
      bad = true;
      nk = nk < 0 ? 0 : cap;
    }
  } else {
    kbase = a.cu_k[b];
    nk = (int64_t)a.cu_k[b + 1] - kbase;
    if (kbase < 0 || nk < 0 || kbase + nk > a.kv_units) {
      bad = true;
      nk = 0;
    }
  }
  if (bad && tid == 0 && blockIdx.x == 0) raise_err(a.err, MKV_DEVERR_TABLE);
  const int64_t shift = nk - nq;  // query t sits at position shift + t
  const int32_t last_q = (qt + kQTok < nq ? qt + kQTok : nq) - 1;  // the workgroup's last
  int64_t kv_end = a.causal ? shift + last_q + 1 : nk;
  if (kv_end > nk) kv_end = nk;
  // this workgroup's key range (the whole range with one split); the last
  // range runs to the sequence's end, so a split_len * splits below the real
  // key count never drops keys
  const int64_t kv_begin = split * (int64_t)a.split_len;
  if (split + 1 < a.splits && kv_begin + a.split_len < kv_end) kv_end = kv_begin + a.split_len;

  // Q as the A operand: row n = query token q0 + n, dims 32 s + 8 g .. +7
  bf16x8 qa[8];
  {
    const bool ok = q0 + n < nq;
    const uint8_t* row = a.q + (((int64_t)qs + q0 + n) * hq + h) * kPRow;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      qa[s] = __builtin_bit_cast(bf16x8, ok ? ld16(row + (32 * s + 8 * g) * 2)
                                            : u32x4{0u, 0u, 0u, 0u});
  }
  // this lane's C rows 4 g + i: query positions, running max and sum
  // and the last key each row sees (keys and positions fit int32: the
  // lengths and offsets are int32)
  float m_run[4], l_run[4];
  int32_t lastk[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m_run[i] = -INFINITY;
    l_run[i] = 0.f;
    const int64_t qpos = shift + q0 + 4 * g + i;
    lastk[i] = (int32_t)(a.causal && qpos < nk - 1 ? qpos : nk - 1);
  }
  f32x4 o[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) o[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int32_t* trow = a.table ? a.table + b * a.tstride : nullptr;

  // K and V of tokens kv0 .. kv0+63 into registers: this thread's 16-byte
  // chunks c = tid + kPThreads u (token c / 32, dims 8 (c % 32) ..); a token
  // past the keys, or on a page outside the pool, is zeros
  u32x4 kreg[kStage], vreg[kStage];
  auto fetch = [&](int64_t kv0) {
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
      const int c = tid + kPThreads * u;
      const int r = c >> 5, col = c & 31;
      const int64_t tok = kv0 + r;
      kreg[u] = vreg[u] = u32x4{0u, 0u, 0u, 0u};
      if (tok < nk) {
        int64_t rowi;
        bool ok = true;
        if (trow) {
          const int32_t page = trow[tok >> 4];
          ok = page >= 0 && page < a.kv_units;
          if (!ok && col == 0) raise_err(a.err, MKV_DEVERR_PAGE);
          rowi = ((int64_t)(ok ? page : 0) * 16 + (tok & 15)) * a.hkv + hk;
        } else {
          rowi = (kbase + tok) * a.hkv + hk;
        }
        if (ok) {
          kreg[u] = ld16(a.k + rowi * kPRow + col * 16);
          vreg[u] = ld16(a.v + rowi * kPRow + col * 16);
        }
      }
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
      const int c = tid + kPThreads * u;
      *reinterpret_cast<u32x4*>(&k_lds[buf][c >> 5][(c & 31) * 8]) = kreg[u];
      *reinterpret_cast<u32x4*>(&v_lds[buf][c >> 5][(c & 31) * 8]) = vreg[u];
    }
  };
  // one barrier per tile: tile i + 1 goes into the buffer that tile i - 1
  // used, which every wave left before the barrier that ended tile i - 1
  if (kv_end > kv_begin) {
    fetch(kv_begin);
    stage(0);
    if (kv_begin + kKvTile < kv_end) fetch(kv_begin + kKvTile);
  }
  __syncthreads();
  int buf = 0;
  for (int64_t kv0 = kv_begin; kv0 < kv_end; kv0 += kKvTile, buf ^= 1) {

    // S = Q K^T for the tile's 16-token quarters: lane holds rows 4 g + i,
    // token 16 q + n
    f32x4 sq[kNQ];
#pragma unroll
    for (int q = 0; q < kNQ; ++q) sq[q] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int q = 0; q < kNQ; ++q) {
        const bf16x8 kk =
            *reinterpret_cast<const bf16x8*>(&k_lds[buf][16 * q + n][32 * s + 8 * g]);
        sq[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[s], kk, sq[q], 0, 0, 0);
      }
    // scores to probabilities in place: token 16 q + n is seen by row 4 g + i
    // when 16 q <= lastk[i] - kv0 - n
    const int32_t kv0i = (int32_t)kv0;
    float alpha[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int32_t rel = lastk[i] - kv0i - n;
      float mx = -INFINITY;
#pragma unroll
      for (int q = 0; q < kNQ; ++q) {
        sq[q][i] = 16 * q <= rel ? sq[q][i] * a.scale_log2 : -INFINITY;
        mx = fmaxf(mx, sq[q][i]);
      }
      mx = row_max16(mx);
      const float m_new = fmaxf(m_run[i], mx);
      const float m_ref = m_new == -INFINITY ? 0.f : m_new;  // a row with nothing seen yet
      alpha[i] = __builtin_amdgcn_exp2f(m_run[i] - m_ref);
      float ps = 0.f;
#pragma unroll
      for (int q = 0; q < kNQ; ++q) {
        sq[q][i] = __builtin_amdgcn_exp2f(sq[q][i] - m_ref);
        ps += sq[q][i];
      }
      ps = row_sum16(ps);
      l_run[i] = l_run[i] * alpha[i] + ps;
      m_run[i] = m_new;
    }
#pragma unroll
    for (int q = 0; q < kNQ; ++q)
      *reinterpret_cast<uint2*>(&p_lds[wave][16 * q + n][4 * g]) =
          uint2{bf16_pack(sq[q][0], sq[q][1]), bf16_pack(sq[q][2], sq[q][3])};
    if (kv0 + kKvTile < kv_end) {  // the next tile into the other buffer; the one after in flight
      stage(buf ^ 1);
      if (kv0 + 2 * kKvTile < kv_end) fetch(kv0 + 2 * kKvTile);
    }
    // rescale only when some row's maximum moved (uniform branch)
    const bool moved = alpha[0] != 1.f || alpha[1] != 1.f || alpha[2] != 1.f || alpha[3] != 1.f;
    if (__builtin_amdgcn_ballot_w64(moved)) {
#pragma unroll
      for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[j][i] *= alpha[i];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // O += P V in 32-token steps: A = P (row n) and B = V (dim 16 j + n) over
    // the same 8 tokens, each by two transposing loads of 4 tokens. The sum
    // runs over the tokens in any order: lane group g takes tokens
    // 32 t + 4 g .. +3 (elements 0-3) and 32 t + 16 + 4 g .. +3 (elements 4-7),
    // so the 32 lanes of one LDS cycle read 8 consecutive rows, whose 32-byte
    // pieces (V rows 544 bytes apart, P rows 32) fall on distinct banks
#pragma unroll
    for (int t = 0; t < kKvTile / 32; ++t) {
      const uint16_t* pbase = &p_lds[wave][32 * t + 4 * g + (n >> 2)][4 * (n & 3)];
      const s16x4 plo = lds_read_tr16(pbase), phi = lds_read_tr16(pbase + 16 * 16);
      const bf16x8 pa = __builtin_bit_cast(
          bf16x8, (short __attribute__((ext_vector_type(8)))){plo.x, plo.y, plo.z, plo.w, phi.x,
                                                              phi.y, phi.z, phi.w});
      const uint16_t* vbase = &v_lds[buf][32 * t + 4 * g + (n >> 2)][4 * (n & 3)];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const s16x4 lo = lds_read_tr16(vbase + 16 * j);
        const s16x4 hi = lds_read_tr16(vbase + 16 * kVStride + 16 * j);
        const bf16x8 vb = __builtin_bit_cast(
            bf16x8, (short __attribute__((ext_vector_type(8)))){lo.x, lo.y, lo.z, lo.w, hi.x,
                                                                   hi.y, hi.z, hi.w});
        o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, vb, o[j], 0, 0, 0);
      }
    }
    __syncthreads();  // tile i + 1 stored; tile i's buffer free for tile i + 2
  }

  // one range: out[token q0 + 4 g + i][h][16 j + n] = O / l (zeros for a row
  // that saw nothing); several: this range's (max, sum, O) for the merge
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int32_t t = q0 + 4 * g + i;
    if (t >= nq) continue;
    const int64_t row = ((int64_t)qs + t) * hq + h;
    if (a.splits == 1) {
      uint16_t* orow = reinterpret_cast<uint16_t*>(a.out + row * kPRow);
      const float L = l_run[i];
#pragma unroll
      for (int j = 0; j < 16; ++j) orow[16 * j + n] = bf16_bits(L > 0.f ? o[j][i] / L : 0.f);
    } else {
      const int64_t at = row * a.splits + split;
#pragma unroll
      for (int j = 0; j < 16; ++j) a.part[at * kPD + 16 * j + n] = o[j][i];
      if (n == 0) {
        a.ml[at * 2] = m_run[i];
        a.ml[at * 2 + 1] = l_run[i];
      }
    }
  }
}

// Combines the key ranges of one query token's KV head: one workgroup of 256
// threads per query t < max_seqlen_q of sequence b (grid.y) and KV head
// (grid.z); its four waves take the head's four query heads, a lane four
// dims (16-byte loads of the fp32 partial rows). It writes exactly the rows
// the attention kernel wrote ranges for: the same query offsets and bounds
// decide, so rows of `out` outside every sequence's queries are left alone,
// as with one range. Each output element is summed over the ranges in range
// order, as a thread per element did (one workgroup per query head was 4x
// the workgroups for the same bytes). Up to 8 ranges, every load
// is issued before the first is used (a loop over the ranges waited a round
// trip per range, twice); loads of ranges past the count are not issued, so
// the bytes read are the ranges' own.
template <int N>
__device__ __forceinline__ void merge_ranges(const float2* ml, const float* part, float& L,
                                             float (&O)[4]) {
  float2 x[N];
  f32x4 p[N];
#pragma unroll
  for (int u = 0; u < N; ++u) {
    x[u] = ml[u];
    p[u] = *reinterpret_cast<const f32x4*>(part + (int64_t)u * kPD);
  }
  float M = -INFINITY;
#pragma unroll
  for (int u = 0; u < N; ++u) M = fmaxf(M, x[u].x);
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const float f = x[u].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(x[u].x - M);
#pragma unroll
    for (int e = 0; e < 4; ++e) O[e] += f * p[u][e];
    L += f * x[u].y;
  }
}

__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a) {
  const int32_t b = blockIdx.y;
  const int32_t qs = a.cu_q[b];
  const int32_t nq_raw = a.cu_q[b + 1] - qs;
  const bool q_ok = qs >= 0 && nq_raw >= 0 && (int64_t)qs + nq_raw <= a.num_q;
  const int32_t nq = q_ok ? (nq_raw < a.max_q ? nq_raw : a.max_q) : 0;
  const int32_t t = blockIdx.x;
  if (t >= nq) return;
  const int64_t row = ((int64_t)qs + t) * ((int64_t)a.hkv * kPG) +
                      (int64_t)blockIdx.z * kPG + (threadIdx.x >> 6);
  const int d = (threadIdx.x & 63) * 4;
  const int64_t at0 = row * a.splits;
  float O[4] = {0.f, 0.f, 0.f, 0.f}, L = 0.f;
  const float2* ml = reinterpret_cast<const float2*>(a.ml) + at0;
  const float* part = a.part + at0 * kPD + d;
  switch (a.splits) {
    case 2: merge_ranges<2>(ml, part, L, O); break;
    case 3: merge_ranges<3>(ml, part, L, O); break;
    case 4: merge_ranges<4>(ml, part, L, O); break;
    case 5: merge_ranges<5>(ml, part, L, O); break;
    case 6: merge_ranges<6>(ml, part, L, O); break;
    case 7: merge_ranges<7>(ml, part, L, O); break;
    case 8: merge_ranges<8>(ml, part, L, O); break;
    default: {  // more than 8 ranges
      float M = -INFINITY;
      for (int sp = 0; sp < a.splits; ++sp) M = fmaxf(M, a.ml[(at0 + sp) * 2]);
      for (int sp = 0; sp < a.splits; ++sp) {
        const float m = a.ml[(at0 + sp) * 2];
        const float f = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
        const f32x4 p = *reinterpret_cast<const f32x4*>(a.part + (at0 + sp) * kPD + d);
#pragma unroll
        for (int e = 0; e < 4; ++e) O[e] += f * p[e];
        L += f * a.ml[(at0 + sp) * 2 + 1];
      }
    }
  }
  uint32_t w[2];
#pragma unroll
  for (int e = 0; e < 2; ++e)
    w[e] = (uint32_t)bf16_bits(L > 0.f ? O[2 * e] / L : 0.f) |
           ((uint32_t)bf16_bits(L > 0.f ? O[2 * e + 1] / L : 0.f) << 16);
  *reinterpret_cast<uint2*>(a.out + row * kPRow + d * 2) = uint2{w[0], w[1]};
}

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int64_t mkv_prefill_attention_workspace_bytes(int64_t num_q_tokens, int32_t num_q_heads,
                                                         int32_t splits) {
  if (num_q_tokens < 0 || num_q_heads <= 0 || splits <= 0) return -1;
  if (splits == 1) return 0;
  return num_q_tokens * num_q_heads * splits * (kPD + 2) * 4;
}

extern "C" int mkv_prefill_attention_bf16(const void* q, const void* k, const void* v,
                                          int64_t kv_units, int32_t num_kv_heads,
                                          int32_t num_q_heads, int32_t head_dim,
                                          const int32_t* page_table, int64_t table_stride,
                                          int32_t table_width, const int32_t* cu_seqlens_q,
                                          const int32_t* cu_seqlens_k, const int32_t* seq_lens_k,
                                          int32_t batch, int64_t num_q_tokens, int32_t max_seqlen_q,
                                          float softmax_scale, int32_t causal, int32_t splits,
                                          int32_t split_len, void* out, void* workspace,
                                          int64_t workspace_bytes, int32_t* err, void* stream) {
  clear_error();
  MKV_REQUIRE(batch >= 0 && kv_units >= 0 && num_kv_heads > 0 && num_q_heads > 0 &&
                  max_seqlen_q >= 0 && num_q_tokens >= 0 && table_width >= 0 &&
                  table_stride >= table_width,
              MKV_E_INVALID, "mkv_prefill_attention_bf16: bad sizes");
  MKV_REQUIRE(head_dim == kPD, MKV_E_UNSUPPORTED,
              "mkv_prefill_attention_bf16: head_dim %d unsupported (256)", head_dim);
  MKV_REQUIRE(num_q_heads == kPG * num_kv_heads, MKV_E_UNSUPPORTED,
              "mkv_prefill_attention_bf16: %d query heads per KV head unsupported (4)",
              num_q_heads / num_kv_heads);
  MKV_REQUIRE(num_q_heads <= 65535 && batch <= 65535, MKV_E_UNSUPPORTED,
              "mkv_prefill_attention_bf16: batch or query heads above 65535");
  MKV_REQUIRE(splits >= 1 && (splits == 1 || (split_len > 0 && split_len % kKvTile == 0)) &&
                  (int64_t)num_kv_heads * splits <= 65535,
              MKV_E_INVALID, "mkv_prefill_attention_bf16: bad key split (%d x %d)", splits,
              split_len);
  if (batch == 0 || max_seqlen_q == 0) return MKV_OK;
  const int64_t need = mkv_prefill_attention_workspace_bytes(num_q_tokens, num_q_heads, splits);
  MKV_REQUIRE(splits == 1 || (workspace && workspace_bytes >= need && aligned16(workspace)),
              MKV_E_INVALID,
              "mkv_prefill_attention_bf16: workspace of %lld bytes (16-byte aligned) required",
              (long long)need);
  MKV_REQUIRE(q && k && v && cu_seqlens_q && out && err &&
                  (page_table ? seq_lens_k != nullptr : cu_seqlens_k != nullptr),
              MKV_E_INVALID, "mkv_prefill_attention_bf16: null pointer");
  MKV_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out), MKV_E_ALIGN,
              "mkv_prefill_attention_bf16: q, k, v and out must be 16-byte aligned");
  PrefillArgs a;
  a.q = static_cast<const uint8_t*>(q);
  a.k = static_cast<const uint8_t*>(k);
  a.v = static_cast<const uint8_t*>(v);
  a.table = page_table;
  a.tstride = table_stride;
  a.twidth = table_width;
  a.kv_units = kv_units;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.lens_k = seq_lens_k;
  a.num_q = num_q_tokens;
  a.max_q = max_seqlen_q;
  a.out = static_cast<uint8_t*>(out);
  a.hkv = num_kv_heads;
  a.causal = causal ? 1 : 0;
  a.splits = splits;
  a.split_len = splits > 1 ? split_len : 0;
  a.part = static_cast<float*>(workspace);
  a.ml = splits > 1 ? a.part + num_q_tokens * num_q_heads * splits * kPD : nullptr;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.err = err;
  const dim3 grid((unsigned)((max_seqlen_q + kQTok - 1) / kQTok), (unsigned)batch,
                  (unsigned)(num_kv_heads * splits));
  hipLaunchKernelGGL(prefill_attn_kernel, grid, dim3(kPThreads), 0, as_stream(stream), a);
  if (splits > 1 && num_q_tokens > 0)
    hipLaunchKernelGGL(prefill_merge_kernel,
                       dim3((unsigned)max_seqlen_q, (unsigned)batch, (unsigned)num_kv_heads),
                       dim3(256), 0, as_stream(stream), a);
  return check_launch("mkv_prefill_attention_bf16");
}
