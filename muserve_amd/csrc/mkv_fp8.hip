// mkv_fp8.hip — bf16 -> fp8 e4m3fn quantize-on-append and fp8 -> bf16
// dequant-gather for gfx950.
//
// A quantisation row is one (token, head) of head_dim = 256 bf16 values. 16
// lanes own a row: each lane loads 32 bytes (16 values), the row absmax is a
// 4-step xor-shuffle inside the 16 lanes, and each lane stores its 16 codes
// with one 16-byte store, so the 256-byte fp8 row is one coalesced store and
// the row's scale one 4-byte store by the group's first lane. On the
// chunked-prefill shape this runs as fast as a plain scattered copy of the
// same bytes: the arithmetic is hidden under the memory traffic.
//
// Exactness: the scale is a correctly rounded fp32 division (hipcc keeps
// division correctly rounded unless fast-math is requested, and this library
// is never built with it); each element's quotient is x * (1/scale) with one
// Markstein correction (div_by_recip in mkv_common.h), equal to x / scale for
// every input the quantiser can see; the clamp propagates NaN like
// torch.clamp. The conversions are gfx950's v_cvt_pk_fp8_f32 (OCP e4m3fn,
// round to nearest even, non-saturating), v_cvt_pk_f32_fp8 and
// v_cvt_pk_bf16_f32, each equal to torch's CPU conversion on every input
// (mkv_check_conversions re-checks them, and the divide, on the device).
#include "mkv_device.h"

namespace mkv {
namespace {

constexpr int kHeadDim = 256;
constexpr int kLanesPerRow = 16;                         // lanes per quantisation row
constexpr int kRowsPerWg = kThreads / kLanesPerRow;      // 16 rows per workgroup
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two fp8 codes (bytes 0-1 or 2-3 of word) times scale, as a packed bf16 pair.
#define dequant2(word, high, scale)                                                       \
  __builtin_bit_cast(uint32_t, __builtin_convertvector(                                   \
      __builtin_amdgcn_cvt_pk_f32_fp8((int)(word), high) * (scale), bf16x2))

struct AppendFp8Args {
  uint8_t* k_pool;
  uint8_t* v_pool;
  float* k_scale;
  float* v_scale;
  int64_t pool_layer_stride;
  int64_t scale_layer_stride;
  int64_t num_slots;
  const uint8_t* k_src;
  const uint8_t* v_src;
  int64_t src_layer_stride;
  int64_t src_token_stride;
  const int64_t* slots;
  uint32_t num_rows;  // tokens * heads
  uint32_t num_heads;
  int32_t* err;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return bits_f32(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return bits_f32(w & 0xffff0000u); }

// torch.clamp(x, -448, 448): NaN passes through unchanged.
__device__ __forceinline__ float clamp448(float x) {
  return x < -448.0f ? -448.0f : (x > 448.0f ? 448.0f : x);
}

// Quantises one 256-value row held as 16 values per lane of a 16-lane group
// and returns the lane's 16 codes, plus the row's scale.
__device__ __forceinline__ u32x4 quantise_row(const u32x4 r0, const u32x4 r1, float& scale_out) {
  const uint32_t w[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
  float x[16];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    x[2 * i] = bf16_lo(w[i]);
    x[2 * i + 1] = bf16_hi(w[i]);
  }
  // absmax over the row. On |x| bit patterns integer max is float max, and
  // any NaN (above +inf as an integer) wins, as torch's amax propagates NaN.
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t ab = f32_bits(x[i]) & 0x7fffffffu;
    m = ab > m ? ab : m;
  }
#pragma unroll
  for (int off = kLanesPerRow / 2; off >= 1; off >>= 1) {
    const uint32_t o = (uint32_t)__shfl_xor((int)m, off, kLanesPerRow);
    m = o > m ? o : m;
  }
  const float amax = bits_f32(m);
  const float clamped = amax < 1e-12f ? 1e-12f : amax;  // .clamp(min=1e-12); NaN stays
  const float scale = clamped / 448.0f;
  const float recip = 1.0f / scale;
  float q[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) q[i] = clamp448(div_by_recip(x[i], scale, recip));
  uint32_t c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[4 * i], q[4 * i + 1], 0, false);
    c[i] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[4 * i + 2], q[4 * i + 3], lo, true);
  }
  scale_out = scale;
  return u32x4{c[0], c[1], c[2], c[3]};
}

// One 16-lane group per (token, head) row of one (layer, K|V): grid.x covers
// the rows, grid.y is layer * 2 + K|V. The source loads do not depend on the
// slot, but the compiler issues them after the slot check; issuing them with
// the slot's load (pinned by an empty asm) measured no faster, the workgroups
// in flight hiding the second round trip. A group whose row is past the end
// exits as a whole, so the shuffles only ever read lanes of the same live row. Source rows are read
// once and pool rows are not read back this step: non-temporal loads and code
// stores, 6 % faster than ordinary ones on the chunked-prefill shape. The
// scales take ordinary stores, 1.3 % faster there than non-temporal ones (a
// page's 16 scales arrive as four 16-byte pieces from four waves). More rows
// per group, K and V in one workgroup, two rows per group, 128- or 512-thread
// workgroups and a persistent grid measured no faster.
// HEADS is the head count when it is 1 or 2 (0: any, read from the
// arguments): a runtime 32-bit division ahead of the first load made the
// one-head launch 10 % slower on the chunked-prefill shape.
template <int HEADS>
__global__ __launch_bounds__(kThreads) void append_fp8_kernel(AppendFp8Args a) {
  const uint32_t lane = threadIdx.x & (kLanesPerRow - 1);
  const uint32_t row = blockIdx.x * kRowsPerWg + threadIdx.x / kLanesPerRow;
  if (row >= a.num_rows) return;
  const uint32_t l = blockIdx.y >> 1;
  const bool is_v = blockIdx.y & 1u;
  const uint32_t nh = HEADS ? (uint32_t)HEADS : a.num_heads;
  const uint32_t t = row / nh;
  const uint32_t h = row - t * nh;
  const int64_t slot = a.slots[t];
  const uint8_t* src = (is_v ? a.v_src : a.k_src) + (int64_t)l * a.src_layer_stride +
                       (int64_t)t * a.src_token_stride + (int64_t)h * (kHeadDim * 2) + lane * 32;
  const u32x4 r0 = ld_nt(src), r1 = ld_nt(src + 16);
  if (slot < 0 || slot >= a.num_slots) {  // -1 skips the token; anything else is an error
    if (slot != -1 && lane == 0 && h == 0 && !is_v) raise_err(a.err, MKV_DEVERR_SLOT);
    return;
  }
  float scale;
  const u32x4 codes = quantise_row(r0, r1, scale);
  uint8_t* pool = (is_v ? a.v_pool : a.k_pool) + (int64_t)l * a.pool_layer_stride;
  st_nt(pool + slot * ((int64_t)nh * kHeadDim) + (int64_t)h * kHeadDim + lane * 16, codes);
  if (lane == 0) {
    float* sp = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(is_v ? a.v_scale : a.k_scale) +
                                         (int64_t)l * a.scale_layer_stride);
    sp[slot * nh + h] = scale;
  }
}

// ---------------------------------------------------------------------------
// dequant-gather: the bf16 gather's tiles with fp8 rows in and bf16 rows out
// (the padding tiles go to the shared gather_pad_kernel). A tile is 4096 fp8
// codes (16 rows of one head, 8 rows of two) and 8 KiB of output; each wave
// owns a contiguous quarter. A lane loads two runs of 8 codes 512 codes apart
// (8-byte non-temporal loads) and writes each as one 16-byte bf16 store, so
// every store instruction of a wave covers 1 KiB of output without gaps.
// Against one 16-byte load and two 16-byte stores per lane (stride-32 store
// addresses), this is 1.3x faster on MI355X; the loads stay non-temporal, the
// stores stay ordinary (both measured faster than the alternatives here).
// ---------------------------------------------------------------------------
constexpr int kDequantThreads = 256;
constexpr int kDequantTileCodes = 4096;

template <int HEADS>
__global__ __launch_bounds__(kDequantThreads) void gather_dequant_kernel(GatherArgs a) {
  constexpr int IN_ROW = HEADS * kHeadDim;           // fp8 bytes per pool row
  constexpr int OUT_ROW = 2 * IN_ROW;                // bf16 bytes per output row
  constexpr int ROWS = kDequantTileCodes / IN_ROW;   // rows per tile
  constexpr int WAVE_CODES = kDequantTileCodes / (kDequantThreads / 64);
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  GatherTile<ROWS> t;
  t.init(a);
  if (t.row0 >= t.nvalid) return;  // padding tile: gather_pad_kernel's
  t.locate(a);
  t.load_pages(a);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c0 = wave * WAVE_CODES + lane * 8;     // first run's code index in the tile
  const int c1 = c0 + WAVE_CODES / 2;              // second run
  const int r0 = c0 / IN_ROW, r1 = c1 / IN_ROW;    // tile rows of the two runs
  const int col = c0 % IN_ROW;                     // same column for both runs
  const int head = col / kHeadDim;
  const uint8_t* plane = (t.is_v ? a.v_pool : a.k_pool) + (int64_t)t.layer * a.pool_layer_stride;
  const float* splane = reinterpret_cast<const float*>(
      reinterpret_cast<const uint8_t*>(t.is_v ? a.v_scale : a.k_scale) +
      (int64_t)t.layer * a.scale_layer_stride);
  uint8_t* out = (t.is_v ? a.v_out : a.k_out) + (int64_t)t.layer * a.out_layer_stride +
                 t.out_row * OUT_ROW;
  u32x2 q0 = u32x2{0u, 0u}, q1 = q0;
  float s0 = 0.0f, s1 = 0.0f;
  if (t.full_data()) {
    const int64_t p0 = t.p0 + r0, p1 = t.p0 + r1;
    const int64_t slot0 = (int64_t)t.page_of(p0) * 16 + (p0 & 15);
    const int64_t slot1 = (int64_t)t.page_of(p1) * 16 + (p1 & 15);
    q0 = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(plane + slot0 * IN_ROW + col));
    q1 = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(plane + slot1 * IN_ROW + col));
    s0 = splane[slot0 * HEADS + head];
    s1 = splane[slot1 * HEADS + head];
    st16(out + 2 * c0, u32x4{dequant2(q0.x, false, s0), dequant2(q0.x, true, s0),
                             dequant2(q0.y, false, s0), dequant2(q0.y, true, s0)});
    st16(out + 2 * c1, u32x4{dequant2(q1.x, false, s1), dequant2(q1.x, true, s1),
                             dequant2(q1.y, false, s1), dequant2(q1.y, true, s1)});
    return;
  }
  // Last data tile (or one with a bad page id): rows past the data are zeros.
  if (t.row0 + r0 < t.nvalid) {
    const int64_t p = t.p0 + r0;
    const int32_t page = t.page_of(p);
    if (page >= 0) {
      const int64_t slot = (int64_t)page * 16 + (p & 15);
      q0 = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(plane + slot * IN_ROW + col));
      s0 = splane[slot * HEADS + head];
    }
  }
  if (t.row0 + r1 < t.nvalid) {
    const int64_t p = t.p0 + r1;
    const int32_t page = t.page_of(p);
    if (page >= 0) {
      const int64_t slot = (int64_t)page * 16 + (p & 15);
      q1 = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(plane + slot * IN_ROW + col));
      s1 = splane[slot * HEADS + head];
    }
  }
  // A zero code times a zero scale is +0, the bytes of a zero row.
  const int64_t row_limit = a.out_offsets ? t.nvalid : a.out_len;
  if (t.row0 + r0 < row_limit)
    st16(out + 2 * c0, u32x4{dequant2(q0.x, false, s0), dequant2(q0.x, true, s0),
                             dequant2(q0.y, false, s0), dequant2(q0.y, true, s0)});
  if (t.row0 + r1 < row_limit)
    st16(out + 2 * c1, u32x4{dequant2(q1.x, false, s1), dequant2(q1.x, true, s1),
                             dequant2(q1.y, false, s1), dequant2(q1.y, true, s1)});
}

template <int HEADS>
int launch_dequant(const GatherArgs& a, int32_t num_layers, hipStream_t stream) {
  constexpr int OUT_ROW = HEADS * kHeadDim * 2;
  constexpr int ROWS = kDequantTileCodes / (HEADS * kHeadDim);
  if (!a.out_offsets)
    hipLaunchKernelGGL((gather_pad_kernel<OUT_ROW, ROWS>), pad_grid(a, OUT_ROW, num_layers),
                       dim3(kPadThreads), 0, stream, a);
  hipLaunchKernelGGL(gather_dequant_kernel<HEADS>, gather_grid(a, ROWS, num_layers),
                     dim3(kDequantThreads), 0, stream, a);
  return check_launch("mkv_gather_dequant_fp8");
}

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int mkv_append_fp8(void* k_pool, void* v_pool, float* k_scale, float* v_scale,
                              int64_t pool_layer_stride, int64_t scale_layer_stride,
                              int64_t num_slots, const void* k_src, const void* v_src,
                              int64_t src_layer_stride, int64_t src_token_stride,
                              const int64_t* slot_mapping, int64_t num_tokens, int32_t num_layers,
                              int32_t num_heads, int32_t head_dim, int32_t* err, void* stream) {
  clear_error();
  MKV_REQUIRE(num_tokens >= 0 && num_layers >= 0 && num_slots >= 0 && num_heads > 0,
              MKV_E_INVALID, "mkv_append_fp8: bad size");
  MKV_REQUIRE(head_dim == kHeadDim, MKV_E_UNSUPPORTED,
              "mkv_append_fp8: head_dim %d unsupported (only 256)", head_dim);
  if (num_tokens == 0 || num_layers == 0) return MKV_OK;
  MKV_REQUIRE(k_pool && v_pool && k_scale && v_scale && k_src && v_src && slot_mapping && err,
              MKV_E_INVALID, "mkv_append_fp8: null pointer");
  MKV_REQUIRE(aligned16(k_src) && aligned16(v_src) && src_layer_stride % 16 == 0 &&
                  src_token_stride % 16 == 0 && aligned16(k_pool) && aligned16(v_pool) &&
                  pool_layer_stride % 16 == 0 && ((uintptr_t)k_scale & 3) == 0 &&
                  ((uintptr_t)v_scale & 3) == 0 && scale_layer_stride % 4 == 0,
              MKV_E_ALIGN, "mkv_append_fp8: misaligned pointer or stride");
  const uint64_t rows = (uint64_t)num_tokens * (uint64_t)num_heads;
  MKV_REQUIRE(rows < (1ull << 31) && num_layers <= 32767, MKV_E_UNSUPPORTED,
              "mkv_append_fp8: too many rows for one call");
  AppendFp8Args a{(uint8_t*)k_pool, (uint8_t*)v_pool, k_scale, v_scale, pool_layer_stride,
                  scale_layer_stride, num_slots, (const uint8_t*)k_src, (const uint8_t*)v_src,
                  src_layer_stride, src_token_stride, slot_mapping, (uint32_t)rows,
                  (uint32_t)num_heads, err};
  dim3 grid((unsigned)((rows + kRowsPerWg - 1) / kRowsPerWg), (unsigned)(2 * num_layers));
  if (num_heads == 1)
    hipLaunchKernelGGL(append_fp8_kernel<1>, grid, dim3(kThreads), 0, as_stream(stream), a);
  else if (num_heads == 2)
    hipLaunchKernelGGL(append_fp8_kernel<2>, grid, dim3(kThreads), 0, as_stream(stream), a);
  else
    hipLaunchKernelGGL(append_fp8_kernel<0>, grid, dim3(kThreads), 0, as_stream(stream), a);
  return check_launch("mkv_append_fp8");
}

extern "C" int mkv_gather_dequant_fp8(const void* k_pool, const void* v_pool, const float* k_scale,
                                      const float* v_scale, int64_t pool_layer_stride,
                                      int64_t scale_layer_stride, int64_t num_pages,
                                      const int32_t* block_tables, int64_t table_stride,
                                      int32_t table_width, const int32_t* seq_lens,
                                      const int32_t* starts, int32_t batch, int64_t out_len,
                                      const int64_t* out_offsets, void* k_out, void* v_out,
                                      int64_t out_layer_stride, int32_t num_layers,
                                      int32_t num_heads, int32_t head_dim, int32_t* err,
                                      void* stream) {
  clear_error();
  MKV_REQUIRE(batch >= 0 && out_len >= 0 && num_layers >= 0 && num_pages >= 0 &&
                  table_width >= 0,
              MKV_E_INVALID, "mkv_gather_dequant_fp8: negative size");
  MKV_REQUIRE(head_dim == kHeadDim && (num_heads == 1 || num_heads == 2), MKV_E_UNSUPPORTED,
              "mkv_gather_dequant_fp8: heads=%d head_dim=%d unsupported (1 or 2 heads of 256)",
              num_heads, head_dim);
  if (batch == 0 || out_len == 0 || num_layers == 0) return MKV_OK;
  MKV_REQUIRE(num_layers <= 32767, MKV_E_UNSUPPORTED, "mkv_gather_dequant_fp8: too many layers for one call");
  MKV_REQUIRE(k_scale && v_scale && scale_layer_stride % 4 == 0, MKV_E_INVALID,
              "mkv_gather_dequant_fp8: bad scale planes");
  GatherArgs a;
  const int rc = fill_gather_args(a, "mkv_gather_dequant_fp8", k_pool, v_pool, pool_layer_stride,
                                  num_pages, block_tables, table_stride, table_width, seq_lens,
                                  starts, batch, out_len, out_offsets, k_out, v_out,
                                  out_layer_stride, num_heads * kHeadDim * 2, err);
  if (rc != MKV_OK) return rc;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.scale_layer_stride = scale_layer_stride;
  hipStream_t s = as_stream(stream);
  return num_heads == 1 ? launch_dequant<1>(a, num_layers, s) : launch_dequant<2>(a, num_layers, s);
}
