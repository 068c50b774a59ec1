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

// Streaming 16-byte store at base + off with cache policy "sc1 nt"
// (device-scope, non-temporal). The global-store builtins can only ask for
// "nt"; a buffer store carries the scope bits too, and on MI355X fills and
// copies stream 3-6 % faster with them. `base` must be the same for the
// whole wave (it becomes a scalar buffer descriptor); `off` is per lane.
// Descriptor: num_records 2^31-1 from base (never clips within a tile),
// word 3 = 32-bit data format, as gfx9-family raw buffer accesses expect.
constexpr int kCpolSc1Nt = 16 | 2;
__device__ __forceinline__ void st_stream(uint8_t* base, uint32_t off, u32x4 v) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(base, (short)0, 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kCpolSc1Nt);
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
  const int64_t* out_offsets;  // packed mode: batch + 1 row offsets
  int64_t out_rows;            // packed mode: rows one layer's output holds
  uint8_t* k_out;
  uint8_t* v_out;
  int64_t out_layer_stride;
  int32_t* err;
};

template <int NP>
__device__ __forceinline__ int32_t pick_page(const int32_t (&pg)[NP], int j) {
  int32_t r = pg[0];
#pragma unroll
  for (int k = 1; k < NP; ++k) r = (j == k) ? pg[k] : r;
  return r;
}

// Tile geometry of the data kernels of the two-kernel gather. A tile is ROWS
// consecutive output rows of one (layer, K|V, sequence); the grid is
// (tile, sequence, layer*2 + K|V), so nothing is decoded by division.
//
// Output rows of a sequence split at data_end = min(roundup(nvalid, ROWS),
// out_len): tiles below it belong to the data kernel (which also zero-fills
// the padding rows of the last, partial tile), rows at or above it to
// gather_pad_kernel<.., ROWS>, so each row is written exactly once.
template <int ROWS>
struct GatherTile {
  static constexpr int NP = (ROWS + 14) / 16 + 1;  // pages ROWS rows can span
  uint32_t b, layer;
  bool is_v;
  int64_t row0, nvalid, data_end, p0, first_page, out_row;
  bool pages_ok;
  int32_t pg[NP];

  // Sequence window (what the padding kernel needs): one or two scalar loads.
  __device__ __forceinline__ void init(const GatherArgs& a) {
    b = blockIdx.y;
    layer = blockIdx.z >> 1;
    is_v = blockIdx.z & 1u;
    row0 = (int64_t)blockIdx.x * ROWS;
    const int64_t len = ld_const(a.seq_lens + b);
    int64_t start = a.starts ? (int64_t)ld_const(a.starts + b) : 0;
    nvalid = len - start;
    nvalid = nvalid < 0 ? 0 : (nvalid > a.out_len ? a.out_len : nvalid);
    if (start < 0) {  // malformed window: padding only, never a negative page
      nvalid = 0;
      start = 0;
    }
    if (a.out_offsets) {
      // packed rows of sequence b stay inside [out_offsets[b], out_offsets[b+1])
      // and inside the output; offsets that leave less room are flagged and
      // the sequence is cut to the room there is (none for a negative start)
      const int64_t o0 = ld_const(a.out_offsets + b);
      int64_t o1 = ld_const(a.out_offsets + b + 1);
      o1 = o1 < a.out_rows ? o1 : a.out_rows;
      const int64_t room = o0 < 0 ? 0 : (o1 > o0 ? o1 - o0 : 0);
      if (room < nvalid || o0 < 0) {
        if (blockIdx.x == 0 && blockIdx.z == 0 && threadIdx.x == 0)
          raise_err(a.err, MKV_DEVERR_TABLE);
        nvalid = room < nvalid ? room : nvalid;
      }
    }
    const int64_t up = (nvalid + ROWS - 1) / ROWS * ROWS;
    data_end = up < a.out_len ? up : a.out_len;
    p0 = start + row0;
    first_page = p0 >> 4;
  }

  // Output row of this tile's first row (padded or packed layout).
  __device__ __forceinline__ void locate(const GatherArgs& a) {
    out_row = (a.out_offsets ? ld_const(a.out_offsets + b) : (int64_t)b * a.out_len) + row0;
  }

  // Page ids of the tile's valid rows (data kernel). All loads are issued
  // before any is inspected; the index is clamped into the table row so an
  // unneeded load stays in bounds. Bad ids become -1 (zero rows) and are
  // reported through the error word.
  __device__ __forceinline__ void load_pages(const GatherArgs& a) {
    const int32_t* row = a.block_tables + (int64_t)b * a.table_stride;
    const int64_t wmax = a.table_width > 0 ? a.table_width - 1 : 0;
    const int64_t end_pos = p0 - row0 + nvalid;  // one past the last valid position
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
      if (pj * 16 < end_pos) {
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

  __device__ __forceinline__ int32_t page_of(int64_t p) const {
    return pick_page(pg, (int)((p >> 4) - first_page));
  }
  __device__ __forceinline__ bool full_data() const { return row0 + ROWS <= nvalid && pages_ok; }
};

// Threads of the padding kernel (one 16-byte store per tile each) and of the
// bf16 data kernel (two 16-byte chunks each); both tiles are 4 KiB of output.
constexpr int kPadThreads = 256;
constexpr int kDataThreads = 128;
constexpr int kTileBytes = kPadThreads * 16;

// Zero-fills the padding rows of a padded gather: rows >= data_end of every
// (layer, K|V, sequence), where data_end rounds the sequence's valid rows up
// to the DATA_ROWS tiles of the data kernel that writes everything below it.
// One 4 KiB tile per workgroup, one 16-byte streaming store per thread, few
// registers: shaped like the fastest fill on MI355X (7.25 TB/s). A workgroup
// that loops over several tiles, or stores several chunks per thread,
// streams measurably slower.
template <int ROW_BYTES, int DATA_ROWS>
__global__ __launch_bounds__(kPadThreads) void gather_pad_kernel(GatherArgs a) {
  constexpr int ROWS = kTileBytes / ROW_BYTES;  // rows per padding tile
  constexpr int RC = ROW_BYTES / 16;
  static_assert(DATA_ROWS % ROWS == 0, "data tiles must be whole padding tiles");
  const uint32_t b = blockIdx.y;
  int64_t nvalid = ld_const(a.seq_lens + b);
  const int64_t start = a.starts ? (int64_t)ld_const(a.starts + b) : 0;
  nvalid = start < 0 ? 0 : nvalid - start;
  nvalid = nvalid < 0 ? 0 : (nvalid > a.out_len ? a.out_len : nvalid);
  const int64_t up = (nvalid + DATA_ROWS - 1) / DATA_ROWS * DATA_ROWS;
  const int64_t data_end = up < a.out_len ? up : a.out_len;
  const int64_t row0 = (int64_t)blockIdx.x * ROWS;
  const int64_t row = row0 + threadIdx.x / RC;
  if (row < data_end || row >= a.out_len) return;
  uint8_t* tile = ((blockIdx.z & 1u) ? a.v_out : a.k_out) +
                  (int64_t)(blockIdx.z >> 1) * a.out_layer_stride +
                  ((int64_t)b * a.out_len + row0) * ROW_BYTES;
  st_stream(tile, threadIdx.x * 16, u32x4{0u, 0u, 0u, 0u});  // row row, chunk threadIdx.x % RC
}

// Grid of the padding kernel (one 4 KiB tile per workgroup).
inline dim3 pad_grid(const GatherArgs& a, int row_bytes, int32_t num_layers) {
  const int64_t rows = kTileBytes / row_bytes;
  return dim3((unsigned)((a.out_len + rows - 1) / rows), a.batch, (unsigned)(2 * num_layers));
}

// Grid of a gather kernel with ROWS-row tiles; 0 tiles when nothing to do.
inline dim3 gather_grid(const GatherArgs& a, int rows, int32_t num_layers) {
  return dim3((unsigned)((a.out_len + rows - 1) / rows), a.batch, (unsigned)(2 * num_layers));
}

// Fills the argument block common to mkv_gather_bf16 and mkv_gather_dequant_fp8.
// out_row_bytes is the size of one output row: in packed mode
// out_layer_stride / out_row_bytes is the capacity of one layer's output.
inline int fill_gather_args(GatherArgs& a, const char* fn, const void* k_pool, const void* v_pool,
                            int64_t pool_layer_stride, int64_t num_pages,
                            const int32_t* block_tables, int64_t table_stride, int32_t table_width,
                            const int32_t* seq_lens, const int32_t* starts, int32_t batch,
                            int64_t out_len, const int64_t* out_offsets, void* k_out, void* v_out,
                            int64_t out_layer_stride, int32_t out_row_bytes, int32_t* err) {
  if (!(k_pool && v_pool && block_tables && seq_lens && k_out && v_out && err))
    return set_error(MKV_E_INVALID, "%s: null pointer", fn);
  if (!(aligned16(k_pool) && aligned16(v_pool) && aligned16(k_out) && aligned16(v_out) &&
        pool_layer_stride % 16 == 0 && out_layer_stride % 16 == 0))
    return set_error(MKV_E_ALIGN, "%s: pointers and strides must be 16-byte aligned", fn);
  if (out_len >= (1ll << 31)) return set_error(MKV_E_UNSUPPORTED, "%s: out_len too large", fn);
  if (out_offsets && out_layer_stride < 0)
    return set_error(MKV_E_INVALID, "%s: negative output capacity", fn);
  if (batch > 65535) return set_error(MKV_E_UNSUPPORTED, "%s: batch %d > 65535", fn, batch);
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
  a.out_rows = out_offsets ? out_layer_stride / out_row_bytes : 0;
  a.k_out = (uint8_t*)k_out;
  a.v_out = (uint8_t*)v_out;
  a.out_layer_stride = out_layer_stride;
  a.err = err;
  return MKV_OK;
}

}  // namespace mkv
