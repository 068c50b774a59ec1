// mkv_fp8.hip — bf16 -> fp8 e4m3fn quantize-on-append and fp8 -> bf16
// dequant-gather for gfx950.
//
// A quantisation row is one (token, head) of head_dim = 256 bf16 values. A
// half-wave (32 lanes) owns a row at a time: each lane holds 16 bytes (8
// values), the row absmax is a 5-step xor-shuffle reduction inside the
// half-wave, and each lane stores 8 fp8 bytes, so the 256-byte fp8 row is one
// coalesced 8-byte-per-lane store. Each half-wave takes 4 rows and loads all
// of them before quantising any, to keep enough bytes in flight.
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

// Quantises one 256-value row held as 8 values per lane of a half-wave and
// returns the lane's 8 codes packed in two words, plus the row's scale.
__device__ __forceinline__ void quantise_row(const u32x4 raw, uint32_t& lo, uint32_t& hi,
                                             float& scale_out) {
  float x[8];
  x[0] = bf16_lo(raw.x); x[1] = bf16_hi(raw.x);
  x[2] = bf16_lo(raw.y); x[3] = bf16_hi(raw.y);
  x[4] = bf16_lo(raw.z); x[5] = bf16_hi(raw.z);
  x[6] = bf16_lo(raw.w); x[7] = bf16_hi(raw.w);
  // absmax over the row. On |x| bit patterns integer max is float max, and
  // any NaN (above +inf as an integer) wins, as torch's amax propagates NaN.
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t ab = f32_bits(x[i]) & 0x7fffffffu;
    m = ab > m ? ab : m;
  }
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) {
    const uint32_t o = (uint32_t)__shfl_xor((int)m, off, 32);
    m = o > m ? o : m;
  }
  const float amax = bits_f32(m);
  const float clamped = amax < 1e-12f ? 1e-12f : amax;  // .clamp(min=1e-12); NaN stays
  const float scale = clamped / 448.0f;
  const float recip = 1.0f / scale;
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = clamp448(div_by_recip(x[i], scale, recip));
  int w0 = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
  w0 = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], w0, true);
  int w1 = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
  w1 = __builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], w1, true);
  lo = (uint32_t)w0;
  hi = (uint32_t)w1;
  scale_out = scale;
}

// A half-wave quantises kRowsPerHalfWave consecutive (token, head) rows of
// one (layer, K|V): all their loads are issued first, so each lane keeps four
// 16-byte loads in flight.
constexpr int kRowsPerHalfWave = 4;
constexpr int kRowsPerWg = (kThreads / 32) * kRowsPerHalfWave;  // 32 rows per workgroup

__global__ __launch_bounds__(kThreads) void append_fp8_kernel(AppendFp8Args a) {
  const uint32_t lane = threadIdx.x & 31u;
  const uint32_t row0 = blockIdx.x * kRowsPerWg + (threadIdx.x >> 5) * kRowsPerHalfWave;
  const uint32_t lkv = blockIdx.y;
  const uint32_t l = lkv >> 1;
  const bool is_v = lkv & 1u;
  const uint8_t* src_base = (is_v ? a.v_src : a.k_src) + (int64_t)l * a.src_layer_stride;
  int64_t slot[kRowsPerHalfWave];
  u32x4 raw[kRowsPerHalfWave];
#pragma unroll
  for (int k = 0; k < kRowsPerHalfWave; ++k) {
    const uint32_t row = row0 + k;
    slot[k] = -1;
    raw[k] = u32x4{0u, 0u, 0u, 0u};
    if (row < a.num_rows) {
      const uint32_t t = row / a.num_heads;
      const uint32_t h = row - t * a.num_heads;
      slot[k] = a.slots[t];
      raw[k] = ld16(src_base + (int64_t)t * a.src_token_stride + (int64_t)h * (kHeadDim * 2) +
                    lane * 16);
    }
  }
  const int64_t row_bytes = (int64_t)a.num_heads * kHeadDim;  // fp8 row of all heads
  uint8_t* pool = (is_v ? a.v_pool : a.k_pool) + (int64_t)l * a.pool_layer_stride;
  float* sp = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(is_v ? a.v_scale : a.k_scale) +
                                       (int64_t)l * a.scale_layer_stride);
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int k = 0; k < kRowsPerHalfWave; ++k) {
    const uint32_t row = row0 + k;
    if (row >= a.num_rows) break;  // the half-wave's rows run out together
    const uint32_t t = row / a.num_heads;
    const uint32_t h = row - t * a.num_heads;
    if (slot[k] < 0 || slot[k] >= a.num_slots) {
      if (slot[k] != -1 && lane == 0 && h == 0 && !is_v) raise_err(a.err, MKV_DEVERR_SLOT);
      continue;
    }
    uint32_t lo, hi;
    float scale;
    quantise_row(raw[k], lo, hi, scale);
    *reinterpret_cast<u32x2*>(pool + slot[k] * row_bytes + (int64_t)h * kHeadDim + lane * 8) =
        u32x2{lo, hi};
    if (lane == 0) sp[slot[k] * a.num_heads + h] = scale;
  }
}

// ---------------------------------------------------------------------------
// dequant-gather: the bf16 gather's tiles with fp8 rows in and bf16 rows out
// (the padding tiles go to the shared gather_pad_kernel). A thread turns 8
// fp8 bytes and its head's scale into 16 output bytes.
// ---------------------------------------------------------------------------
// One thread per 16 fp8 bytes (one 16-byte load, two 16-byte stores) and 256
// threads per tile: the shape that streamed fastest on MI355X.
constexpr int kDequantThreads = 256;

template <int HEADS>
__global__ __launch_bounds__(kDequantThreads) void gather_dequant_kernel(GatherArgs a) {
  constexpr int OUT_ROW = HEADS * kHeadDim * 2;  // bf16 bytes per output row
  constexpr int IN_ROW = HEADS * kHeadDim;       // fp8 bytes per pool row
  constexpr int RC = IN_ROW / 16;                // 16-byte fp8 chunks per row
  constexpr int ROWS = kDequantThreads / RC;     // one chunk per thread
  GatherTile<ROWS> t;
  t.init(a);
  if (t.row0 >= t.nvalid) return;  // padding tile: gather_pad_kernel's
  t.locate(a);
  t.load_pages(a);
  const int col = threadIdx.x % RC;
  const int head = col / (kHeadDim / 16);
  const int r = threadIdx.x / RC;
  const uint8_t* plane = (t.is_v ? a.v_pool : a.k_pool) + (int64_t)t.layer * a.pool_layer_stride;
  const float* splane = reinterpret_cast<const float*>(
      reinterpret_cast<const uint8_t*>(t.is_v ? a.v_scale : a.k_scale) +
      (int64_t)t.layer * a.scale_layer_stride);
  uint8_t* out = (t.is_v ? a.v_out : a.k_out) + (int64_t)t.layer * a.out_layer_stride +
                 (t.out_row + r) * OUT_ROW + col * 32;
  u32x4 o0 = u32x4{0u, 0u, 0u, 0u}, o1 = o0;
  if (t.row0 + r < t.nvalid) {
    const int64_t p = t.p0 + r;
    const int32_t page = t.page_of(p);
    if (page >= 0) {
      const int64_t slot = (int64_t)page * 16 + (p & 15);
      const u32x4 q = ld_nt(plane + slot * IN_ROW + col * 16);
      const float s = splane[slot * HEADS + head];
      o0 = u32x4{dequant2(q.x, false, s), dequant2(q.x, true, s), dequant2(q.y, false, s),
                 dequant2(q.y, true, s)};
      o1 = u32x4{dequant2(q.z, false, s), dequant2(q.z, true, s), dequant2(q.w, false, s),
                 dequant2(q.w, true, s)};
    }
  }
  if (t.row0 + r < (a.out_offsets ? t.nvalid : a.out_len)) {
    st_nt(out, o0);
    st_nt(out + 16, o1);
  }
}

template <int HEADS>
int launch_dequant(const GatherArgs& a, int32_t num_layers, hipStream_t stream) {
  constexpr int OUT_ROW = HEADS * kHeadDim * 2;
  constexpr int ROWS = kDequantThreads / (HEADS * kHeadDim / 16);
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
  hipLaunchKernelGGL(append_fp8_kernel, grid, dim3(kThreads), 0, as_stream(stream), a);
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
                                  out_layer_stride, err);
  if (rc != MKV_OK) return rc;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.scale_layer_stride = scale_layer_stride;
  hipStream_t s = as_stream(stream);
  return num_heads == 1 ? launch_dequant<1>(a, num_layers, s) : launch_dequant<2>(a, num_layers, s);
}
