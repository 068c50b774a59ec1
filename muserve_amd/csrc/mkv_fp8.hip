// mkv_fp8.hip — bf16 -> fp8 e4m3fn quantize-on-append and fp8 -> bf16
// dequant-gather for gfx950.
//
// A quantisation row is one (token, head) of head_dim = 256 bf16 values. A
// half-wave (32 lanes) owns a row: each lane loads 16 bytes (8 values), the
// row absmax is a 5-step xor-shuffle reduction inside the half-wave, and each
// lane stores 8 fp8 bytes, so the 256-byte fp8 row is written by one
// coalesced 8-byte-per-lane store.
//
// Exactness: the scale and the per-element quotient use IEEE fp32 division
// (hipcc keeps division correctly rounded unless fast-math is requested,
// and this library is never built with it), the clamp propagates NaN like
// torch.clamp, and the e4m3fn encoder is the integer RNE in mkv_common.h.
#include "mkv_device.h"

namespace mkv {
namespace {

constexpr int kHeadDim = 256;
constexpr int kRowsPerWg = kThreads / 32;  // 8 quantisation rows per workgroup

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

__global__ __launch_bounds__(kThreads) void append_fp8_kernel(AppendFp8Args a) {
  const uint32_t row = blockIdx.x * kRowsPerWg + (threadIdx.x >> 5);
  const uint32_t lane = threadIdx.x & 31u;
  if (row >= a.num_rows) return;  // whole half-waves leave together
  const uint32_t t = row / a.num_heads;
  const uint32_t h = row - t * a.num_heads;
  const uint32_t lkv = blockIdx.y;
  const uint32_t l = lkv >> 1;
  const bool is_v = lkv & 1u;
  const int64_t slot = a.slots[t];
  if (slot < 0 || slot >= a.num_slots) {
    if (slot != -1 && lane == 0 && h == 0 && !is_v) raise_err(a.err, MKV_DEVERR_SLOT);
    return;
  }
  const uint8_t* src = (is_v ? a.v_src : a.k_src) + (int64_t)l * a.src_layer_stride +
                       (int64_t)t * a.src_token_stride + (int64_t)h * (kHeadDim * 2) + lane * 16;
  const u32x4 raw = ld16(src);
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

  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) lo |= (uint32_t)f32_to_e4m3fn(clamp448(x[i] / scale)) << (8 * i);
#pragma unroll
  for (int i = 0; i < 4; ++i) hi |= (uint32_t)f32_to_e4m3fn(clamp448(x[4 + i] / scale)) << (8 * i);

  const int64_t row_bytes = (int64_t)a.num_heads * kHeadDim;  // fp8 row of all heads
  uint8_t* dst = (is_v ? a.v_pool : a.k_pool) + (int64_t)l * a.pool_layer_stride +
                 slot * row_bytes + (int64_t)h * kHeadDim + lane * 8;
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  *reinterpret_cast<u32x2*>(dst) = u32x2{lo, hi};
  if (lane == 0) {
    float* sp = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(is_v ? a.v_scale : a.k_scale) +
                                         (int64_t)l * a.scale_layer_stride);
    sp[slot * a.num_heads + h] = scale;
  }
}

// ---------------------------------------------------------------------------
// dequant-gather: the bf16 gather's tiles with fp8 rows in and bf16 rows out
// (the padding tiles go to the shared gather_pad_kernel). A thread turns 8
// fp8 bytes and its head's scale into 16 output bytes.
// ---------------------------------------------------------------------------
template <int HEADS>
__global__ __launch_bounds__(kDataThreads) void gather_dequant_kernel(GatherArgs a) {
  constexpr int OUT_ROW = HEADS * kHeadDim * 2;  // bf16 bytes per output row
  constexpr int IN_ROW = HEADS * kHeadDim;       // fp8 bytes per pool row
  constexpr int ROWS = kTileBytes / OUT_ROW;
  constexpr int RC = OUT_ROW / 16;               // output chunks per row
  constexpr int RSTEP = kDataThreads / RC;
  constexpr int CPT = ROWS * RC / kDataThreads;
  static_assert(RC * RSTEP == kDataThreads && CPT * kDataThreads == ROWS * RC, "tile shape");
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  GatherTile<ROWS> t;
  t.init(a);
  if (t.row0 >= t.nvalid) return;  // padding tile: gather_pad_kernel's
  t.locate(a);
  t.load_pages(a);
  const int col = threadIdx.x % RC;
  const int head = col / (kHeadDim / 8);
  const int rsub = threadIdx.x / RC;
  const uint8_t* plane = (t.is_v ? a.v_pool : a.k_pool) + (int64_t)t.layer * a.pool_layer_stride;
  const float* splane = reinterpret_cast<const float*>(
      reinterpret_cast<const uint8_t*>(t.is_v ? a.v_scale : a.k_scale) +
      (int64_t)t.layer * a.scale_layer_stride);
  uint8_t* out = (t.is_v ? a.v_out : a.k_out) + (int64_t)t.layer * a.out_layer_stride +
                 t.out_row * OUT_ROW + col * 16;

  u32x2 q[CPT];
  float s[CPT];
  bool valid[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int r = rsub + i * RSTEP;
    valid[i] = false;
    q[i] = u32x2{0u, 0u};
    s[i] = 0.0f;
    if (t.row0 + r < t.nvalid) {
      const int64_t p = t.p0 + r;
      const int32_t page = t.page_of(p);
      if (page >= 0) {
        const int64_t slot = (int64_t)page * 16 + (p & 15);
        q[i] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x2*>(plane + slot * IN_ROW + col * 8));
        s[i] = splane[slot * HEADS + head];
        valid[i] = true;
      }
    }
  }
  const int64_t row_limit = a.out_offsets ? t.nvalid : a.out_len;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int r = rsub + i * RSTEP;
    u32x4 o = u32x4{0u, 0u, 0u, 0u};
    if (valid[i]) {
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t word = k < 2 ? q[i].x : q[i].y;
        const uint32_t b0 = (word >> (16 * (k & 1))) & 0xffu;
        const uint32_t b1 = (word >> (16 * (k & 1) + 8)) & 0xffu;
        const uint32_t e0 = f32_to_bf16_rne(e4m3fn_to_f32(b0) * s[i]);
        const uint32_t e1 = f32_to_bf16_rne(e4m3fn_to_f32(b1) * s[i]);
        w[k] = e0 | (e1 << 16);
      }
      o = u32x4{w[0], w[1], w[2], w[3]};
    }
    if (t.row0 + r < row_limit) st_nt(out + (int64_t)r * OUT_ROW, o);
  }
}

template <int HEADS>
int launch_dequant(const GatherArgs& a, int32_t num_layers, hipStream_t stream) {
  constexpr int OUT_ROW = HEADS * kHeadDim * 2;
  const dim3 grid = gather_grid(a, kTileBytes / OUT_ROW, num_layers);
  if (!a.out_offsets)
    hipLaunchKernelGGL(gather_pad_kernel<OUT_ROW>, grid, dim3(kPadThreads), 0, stream, a);
  hipLaunchKernelGGL(gather_dequant_kernel<HEADS>, grid, dim3(kDataThreads), 0, stream, a);
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
