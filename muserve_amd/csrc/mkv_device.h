// mkv_device.h — device-side pieces shared by the gfx950 kernels: 16-byte
// vector I/O, the device error word, and the gather-tile resolver used by
// both the bf16 gather and the fp8 dequant-gather.
#pragma once

#include "mkv_common.h"
#include "mkv_host.h"

namespace mkv {

__device__ __forceinline__ u32x4 ld_nt(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st_nt(uint8_t* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}
__device__ __forceinline__ u32x4 ld16(const uint8_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st16(uint8_t* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}
// Workgroup-uniform read-only metadata (sequence lengths, window starts, page
// ids): reading through the constant address space lets the compiler use
// scalar loads. The memory is written only by earlier launches, and the
// scalar cache is invalidated at every dispatch.
template <typename T>
__device__ __forceinline__ T ld_const(const T* p) {
  return *(const __attribute__((address_space(4))) T*)(p);
}

// Device error bits go through a vector-memory atomic on the caller's word.
__device__ __forceinline__ void raise_err(int32_t* err, int32_t bit) { atomicOr(err, bit); }

// Arguments of a block-table gather (see mkv_gather_bf16 in mkv.h). Row
// geometry is a template parameter of each kernel, not an argument.
struct GatherArgs {
  const uint8_t* k_pool;
  const uint8_t* v_pool;
  const float* k_scale;  // fp8 dequant-gather only
  const float* v_scale;
  int64_t pool_layer_stride;
  int64_t scale_layer_stride;
  int64_t num_pages;
  const int32_t* block_tables;
  int64_t table_stride;
  int32_t table_width;
  const int32_t* seq_lens;
  const int32_t* starts;
  uint32_t batch;
  int64_t out_len;
  const int64_t* out_offsets;
  uint8_t* k_out;
  uint8_t* v_out;
  int64_t out_layer_stride;
  uint32_t tiles_per_seq;
  uint64_t total_tiles;
  int32_t* err;
};

template <int NP>
__device__ __forceinline__ int32_t pick_page(const int32_t (&pg)[NP], int j) {
  int32_t r = pg[0];
#pragma unroll
  for (int k = 1; k < NP; ++k) r = (j == k) ? pg[k] : r;
  return r;
}

// One gather tile = ROWS consecutive output rows of one (layer, K|V,
// sequence). Everything here depends only on the tile id and on scalar loads,
// so it stays in scalar registers; pg[] holds the (at most NP) page ids the
// tile's valid rows live in, -1 where a row must be zero.
template <int ROWS>
struct GatherTile {
  static constexpr int NP = (ROWS + 14) / 16 + 1;
  uint32_t lkv, b;
  int64_t row0, nvalid, p0, first_page, out_row;
  bool skip;
  bool pages_ok;  // every page a valid row needs resolved to a real page id
  int32_t pg[NP];

  __device__ __forceinline__ void init(const GatherArgs& a, uint64_t tile_id) {
    const uint32_t tile = (uint32_t)(tile_id % a.tiles_per_seq);
    const uint64_t rest = tile_id / a.tiles_per_seq;
    b = (uint32_t)(rest % a.batch);
    lkv = (uint32_t)(rest / a.batch);
    const bool packed = a.out_offsets != nullptr;
    const int64_t len = ld_const(a.seq_lens + b);
    int64_t start = a.starts ? (int64_t)ld_const(a.starts + b) : 0;
    const int64_t out_base = packed ? ld_const(a.out_offsets + b) : (int64_t)b * a.out_len;
    nvalid = len - start;
    nvalid = nvalid < 0 ? 0 : (nvalid > a.out_len ? a.out_len : nvalid);
    if (start < 0) {  // malformed window: emit padding only, never a negative page
      nvalid = 0;
      start = 0;
    }
    row0 = (int64_t)tile * ROWS;
    skip = packed && row0 >= nvalid;
    out_row = out_base + row0;
    p0 = start + row0;
    first_page = p0 >> 4;
    const int64_t end_pos = start + nvalid;  // one past the last valid position
    // Issue every page-id load before inspecting any: the index is clamped
    // into the table row so an unneeded load stays in bounds.
    const int32_t* row = a.block_tables + (int64_t)b * a.table_stride;
    const int64_t wmax = a.table_width > 0 ? a.table_width - 1 : 0;
    int32_t raw[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const int64_t pj = first_page + j;
      raw[j] = a.table_width > 0 ? ld_const(row + (pj < wmax ? pj : wmax)) : -1;
    }
    int32_t bad = 0;
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const int64_t pj = first_page + j;
      int32_t page = -1;
      if (!skip && pj * 16 < end_pos) {
        if (pj >= a.table_width) {
          bad |= MKV_DEVERR_TABLE;
        } else if (raw[j] < 0 || raw[j] >= a.num_pages) {
          bad |= MKV_DEVERR_PAGE;
        } else {
          page = raw[j];
        }
      }
      pg[j] = page;
    }
    pages_ok = bad == 0;
    if (bad && threadIdx.x == 0) raise_err(a.err, bad);
  }

  // All ROWS rows hold data from valid pages: straight-line loads and stores.
  __device__ __forceinline__ bool full_data() const { return row0 + ROWS <= nvalid && pages_ok; }
  // All ROWS rows are padding inside the output: straight-line zero stores.
  __device__ __forceinline__ bool full_pad(int64_t out_len) const {
    return row0 >= nvalid && row0 + ROWS <= out_len;
  }

  // Page of output row r of this tile (valid rows only).
  __device__ __forceinline__ int32_t page_of(int64_t p) const {
    return pick_page(pg, (int)((p >> 4) - first_page));
  }
};

// Largest grid a gather launches; bigger jobs loop over tiles inside it.
constexpr uint64_t kMaxGridWgs = 1u << 22;

// Fills the argument block common to mkv_gather_bf16 and mkv_gather_dequant_fp8.
inline int fill_gather_args(GatherArgs& a, const char* fn, const void* k_pool, const void* v_pool,
                            int64_t pool_layer_stride, int64_t num_pages,
                            const int32_t* block_tables, int64_t table_stride, int32_t table_width,
                            const int32_t* seq_lens, const int32_t* starts, int32_t batch,
                            int64_t out_len, const int64_t* out_offsets, void* k_out, void* v_out,
                            int64_t out_layer_stride, int32_t* err) {
  if (!(k_pool && v_pool && block_tables && seq_lens && k_out && v_out && err))
    return set_error(MKV_E_INVALID, "%s: null pointer", fn);
  if (!(aligned16(k_pool) && aligned16(v_pool) && aligned16(k_out) && aligned16(v_out) &&
        pool_layer_stride % 16 == 0 && out_layer_stride % 16 == 0))
    return set_error(MKV_E_ALIGN, "%s: pointers and strides must be 16-byte aligned", fn);
  if (out_len >= (1ll << 40)) return set_error(MKV_E_UNSUPPORTED, "%s: out_len too large", fn);
  a = GatherArgs{};
  a.k_pool = (const uint8_t*)k_pool;
  a.v_pool = (const uint8_t*)v_pool;
  a.pool_layer_stride = pool_layer_stride;
  a.num_pages = num_pages;
  a.block_tables = block_tables;
  a.table_stride = table_stride;
  a.table_width = table_width;
  a.seq_lens = seq_lens;
  a.starts = starts;
  a.batch = (uint32_t)batch;
  a.out_len = out_len;
  a.out_offsets = out_offsets;
  a.k_out = (uint8_t*)k_out;
  a.v_out = (uint8_t*)v_out;
  a.out_layer_stride = out_layer_stride;
  a.err = err;
  return MKV_OK;
}

}  // namespace mkv
