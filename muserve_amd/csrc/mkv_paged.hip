// mkv_paged.hip — paged-pool append, block-table gather, decode-step slot
// assignment and page copies for gfx950.
//
// The pool keeps the reference layout [L, 2, P, 16, H, D]
// (muserve/kv_cache.py:45-49): one (layer, K|V) plane is an array of P*16
// token rows, and a page is 16 consecutive rows (8 KiB for one bf16 head of
// 256). Every kernel here is a pure byte mover, so the design goal is HBM
// streaming efficiency: 16-byte vector accesses, consecutive lanes on
// consecutive addresses, all loads of a thread issued before its stores, and
// non-temporal hints on data that is not re-read within the step.
//
// A padded gather is two launches: a write-only padding kernel shaped like a
// fill (one 16-byte store per thread, few registers, so full occupancy) and a
// data kernel for the rows that exist. Fused into one kernel the padding
// tiles carried the data path's registers and latency and the whole gather
// ran about 10 points of HBM peak slower.
#include "mkv_device.h"

namespace mkv {
namespace {

// ---------------------------------------------------------------------------
// append: one thread per 16-byte chunk of a (layer, K|V, token) row.
// ---------------------------------------------------------------------------
struct AppendArgs {
  uint8_t* k_pool;
  uint8_t* v_pool;
  int64_t pool_layer_stride;
  int64_t num_slots;
  const uint8_t* k_src;
  const uint8_t* v_src;
  int64_t src_layer_stride;
  int64_t src_token_stride;
  const int64_t* slots;
  uint32_t num_tokens;
  uint32_t row_chunks;
  int32_t* err;
};

// RC: 16-byte chunks per row when the row is one bf16 head of 256 (32),
// 0 for any other row size, read from the arguments (a runtime division).
template <int RC>
__global__ __launch_bounds__(kThreads) void append_rows_kernel(AppendArgs a) {
  const uint32_t g = blockIdx.x * kThreads + threadIdx.x;
  const uint32_t rc = RC ? (uint32_t)RC : a.row_chunks;
  const uint32_t t = g / rc;
  if (t >= a.num_tokens) return;
  const uint32_t col = g - t * rc;
  const uint32_t lkv = blockIdx.y;  // layer*2 + (0: K, 1: V)
  const uint32_t l = lkv >> 1;
  const bool is_v = lkv & 1u;
  const int64_t slot = a.slots[t];
  if (slot < 0 || slot >= a.num_slots) {
    if (slot != -1 && col == 0 && !is_v) raise_err(a.err, MKV_DEVERR_SLOT);
    return;
  }
  const int64_t row_bytes = (int64_t)rc * 16;
  const uint8_t* src = (is_v ? a.v_src : a.k_src) + (int64_t)l * a.src_layer_stride +
                       (int64_t)t * a.src_token_stride + (int64_t)col * 16;
  uint8_t* dst = (is_v ? a.v_pool : a.k_pool) + (int64_t)l * a.pool_layer_stride +
                 slot * row_bytes + (int64_t)col * 16;
  st16(dst, ld16(src));
}

// ---------------------------------------------------------------------------
// gather, data part: one 4 KiB tile of one (layer, K|V, sequence) per
// workgroup of 128 threads; each thread issues both of its 16-byte loads
// before either store. Tiles past the sequence's data belong to
// gather_pad_kernel (mkv_device.h) and return at once.
// ---------------------------------------------------------------------------
template <int ROW_BYTES>
__global__ __launch_bounds__(kDataThreads) void gather_data_kernel(GatherArgs a) {
  constexpr int ROWS = kTileBytes / ROW_BYTES;
  constexpr int RC = ROW_BYTES / 16;            // 16-byte chunks per row
  constexpr int RSTEP = kDataThreads / RC;      // rows between a thread's chunks
  constexpr int CPT = ROWS * RC / kDataThreads; // chunks per thread
  static_assert(CPT * kDataThreads == ROWS * RC && RSTEP * RC == kDataThreads, "tile shape");
  GatherTile<ROWS> t;
  t.init(a);
  if (t.row0 >= t.nvalid) return;
  t.locate(a);
  t.load_pages(a);
  const int col = threadIdx.x % RC;
  const int rsub = threadIdx.x / RC;
  const uint8_t* plane = (t.is_v ? a.v_pool : a.k_pool) + (int64_t)t.layer * a.pool_layer_stride;
  uint8_t* tile = (t.is_v ? a.v_out : a.k_out) + (int64_t)t.layer * a.out_layer_stride +
                  t.out_row * ROW_BYTES;
  u32x4 v[CPT];
  if (t.full_data()) {
    // Straight-line: the waitcnt pass can overlap the stores (vmcnt counts
    // stores as well as loads, so a per-row guard would serialise them).
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int64_t p = t.p0 + rsub + i * RSTEP;
      v[i] = ld_nt(plane + ((int64_t)t.page_of(p) * 16 + (p & 15)) * ROW_BYTES + col * 16);
    }
#pragma unroll
    for (int i = 0; i < CPT; ++i) st_stream(tile, (rsub + i * RSTEP) * ROW_BYTES + col * 16, v[i]);
    return;
  }
  // Last data tile (or one with a bad page id): per-row guards.
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int r = rsub + i * RSTEP;
    v[i] = u32x4{0u, 0u, 0u, 0u};
    if (t.row0 + r < t.nvalid) {
      const int64_t p = t.p0 + r;
      const int32_t page = t.page_of(p);
      if (page >= 0)
        v[i] = ld_nt(plane + ((int64_t)page * 16 + (p & 15)) * ROW_BYTES + col * 16);
    }
  }
  const int64_t row_limit = a.out_offsets ? t.nvalid : a.out_len;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int r = rsub + i * RSTEP;
    if (t.row0 + r < row_limit) st_stream(tile, r * ROW_BYTES + col * 16, v[i]);
  }
}

template <int ROW_BYTES>
int launch_gather(const GatherArgs& a, int32_t num_layers, hipStream_t stream) {
  constexpr int ROWS = kTileBytes / ROW_BYTES;
  if (!a.out_offsets)  // padded layout: zero tiles first, then the data tiles
    hipLaunchKernelGGL((gather_pad_kernel<ROW_BYTES, ROWS>), pad_grid(a, ROW_BYTES, num_layers),
                       dim3(kPadThreads), 0, stream, a);
  hipLaunchKernelGGL(gather_data_kernel<ROW_BYTES>, gather_grid(a, ROWS, num_layers),
                     dim3(kDataThreads), 0, stream, a);
  return check_launch("mkv_gather_bf16");
}

// ---------------------------------------------------------------------------
// decode-step slot assignment, one thread per sequence.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void decode_slots_kernel(
    int32_t* seq_lens, int32_t* bt, int64_t stride, int32_t width, const int32_t* new_pages,
    int32_t batch, int64_t num_pages, int64_t* slot_out, int32_t* err) {
  const int b = blockIdx.x * kThreads + threadIdx.x;
  if (b >= batch) return;
  const int32_t len = seq_lens[b];
  const int32_t j = len >> 4, off = len & 15;
  if (len < 0 || j >= width) {
    raise_err(err, MKV_DEVERR_TABLE);
    slot_out[b] = -1;
    return;
  }
  int32_t page;
  if (off == 0) {
    page = new_pages[b];
    if (page < 0 || page >= num_pages) {
      raise_err(err, page < 0 ? MKV_DEVERR_NEW_PAGE : MKV_DEVERR_PAGE);
      slot_out[b] = -1;
      return;
    }
    bt[(int64_t)b * stride + j] = page;
  } else {
    page = bt[(int64_t)b * stride + j];
    if (page < 0 || page >= num_pages) {
      raise_err(err, MKV_DEVERR_PAGE);
      slot_out[b] = -1;
      return;
    }
  }
  slot_out[b] = (int64_t)page * 16 + off;
  seq_lens[b] = len + 1;
}

// ---------------------------------------------------------------------------
// scheduler step plan: one workgroup per batch entry (a decode token or a
// prefill chunk). Nothing an entry reads is written by another entry (rows are
// unique per step), and an entry's own new pages are taken from new_pages
// rather than read back from the table it writes, so no barrier is needed.
// ---------------------------------------------------------------------------
struct StepPlanArgs {
  int32_t* tables;  // persistent [num_rows, stride] rows
  int64_t stride;
  int32_t width;
  int32_t num_rows;
  const MkvStepEntry* entries;
  int32_t num_entries;
  const int32_t* new_pages;
  int32_t num_new_pages;
  int64_t num_pages;
  int64_t* slot_out;
  int64_t* pos_out;
  int64_t num_tokens;
  int32_t* step_tables;  // [num_entries, step_stride], may be null
  int64_t step_stride;
  int32_t step_width;
  int32_t* step_lens;
  int32_t* rows_out;
  int64_t* cu_seqlens;
  int32_t* err;
};

__global__ __launch_bounds__(kThreads) void step_plan_kernel(StepPlanArgs a) {
  const int32_t i = blockIdx.x;
  const MkvStepEntry e = a.entries[i];
  const int64_t next = (i + 1 < a.num_entries) ? (int64_t)a.entries[i + 1].tok_off : a.num_tokens;
  // Token offsets must tile [0, num_tokens) in entry order; otherwise this
  // entry's output range is unknown and nothing of it is written.
  const bool offsets_ok = e.count >= 0 && e.tok_off >= 0 && (i > 0 || e.tok_off == 0) &&
                          (int64_t)e.tok_off + e.count == next && next <= a.num_tokens;
  const int64_t pages = (int64_t)e.held + e.new_pages;
  const bool ok = offsets_ok && e.row >= 0 && e.row < a.num_rows && e.start >= 0 &&
                  e.held >= 0 && e.new_pages >= 0 && pages <= a.width &&
                  (int64_t)e.start + e.count <= pages * 16 && e.page_off >= 0 &&
                  (int64_t)e.page_off + e.new_pages <= a.num_new_pages &&
                  (!a.step_tables || pages <= a.step_width);
  if (!ok) {
    if (threadIdx.x == 0) {
      raise_err(a.err, MKV_DEVERR_TABLE);
      a.step_lens[i] = 0;
      a.rows_out[i] = -1;
      if (offsets_ok) a.cu_seqlens[i] = e.tok_off;
    }
    if (offsets_ok)
      for (int32_t t = threadIdx.x; t < e.count; t += kThreads) {
        a.slot_out[e.tok_off + t] = -1;
        a.pos_out[e.tok_off + t] = (int64_t)e.start + t;
      }
    if (a.step_tables)
      for (int32_t j = threadIdx.x; j < a.step_width; j += kThreads)
        a.step_tables[(int64_t)i * a.step_stride + j] = 0;
    return;
  }
  int32_t* row = a.tables + (int64_t)e.row * a.stride;
  const int32_t* fresh = a.new_pages + e.page_off;
  auto page_at = [&](int32_t j) -> int32_t {  // page j of the row after this step
    const int32_t p = j < e.held ? row[j] : fresh[j - e.held];
    return (p >= 0 && p < a.num_pages) ? p : -1;
  };
  int32_t bad = 0;
  for (int32_t j = threadIdx.x; j < e.new_pages; j += kThreads) {
    const int32_t p = fresh[j];
    if (p < 0 || p >= a.num_pages) bad = MKV_DEVERR_PAGE;
    row[e.held + j] = (p >= 0 && p < a.num_pages) ? p : -1;
  }
  for (int32_t t = threadIdx.x; t < e.count; t += kThreads) {
    const int64_t pos = (int64_t)e.start + t;
    const int32_t p = page_at((int32_t)(pos >> 4));
    if (p < 0) bad = MKV_DEVERR_PAGE;
    a.slot_out[e.tok_off + t] = p < 0 ? -1 : (int64_t)p * 16 + (pos & 15);
    a.pos_out[e.tok_off + t] = pos;
  }
  if (a.step_tables) {
    // the reference's page-table tensor: the row's pages, then zeros
    // (muserve/kv_cache.py:149-158)
    int32_t* out = a.step_tables + (int64_t)i * a.step_stride;
    for (int32_t j = threadIdx.x; j < a.step_width; j += kThreads) {
      int32_t p = 0;
      if (j < pages) {
        p = page_at(j);
        if (p < 0) bad = MKV_DEVERR_PAGE;
      }
      out[j] = p;
    }
  }
  if (threadIdx.x == 0) {
    a.step_lens[i] = e.start + e.count;
    a.rows_out[i] = e.row;
    a.cu_seqlens[i] = e.tok_off;
    if (i + 1 == a.num_entries) a.cu_seqlens[i + 1] = (int64_t)e.tok_off + e.count;
  }
  if (bad) raise_err(a.err, bad);
}

// ---------------------------------------------------------------------------
// page copies: one workgroup per (pair, plane) on a 2-D grid.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void copy_pages_kernel(
    uint8_t* pool, int64_t plane_stride, int64_t num_pages, int64_t page_bytes,
    const int32_t* src, const int32_t* dst, int32_t* err) {
  const uint32_t i = blockIdx.x, q = blockIdx.y;  // pair, plane
  const int32_t s = src[i], d = dst[i];
  if (s < 0 || d < 0) return;  // a negative id marks "no copy" for this pair
  if (s >= num_pages || d >= num_pages) {
    if (threadIdx.x == 0 && q == 0) raise_err(err, MKV_DEVERR_PAGE);
    return;
  }
  const uint8_t* sp = pool + q * plane_stride + (int64_t)s * page_bytes;
  uint8_t* dp = pool + q * plane_stride + (int64_t)d * page_bytes;
  const int64_t chunks = page_bytes / 16;
  const uint32_t o0 = threadIdx.x * 16, o1 = (threadIdx.x + kThreads) * 16;
  if (chunks == 2 * kThreads) {  // an 8 KiB page (bf16, 1 head of 256): straight-line
    const u32x4 v0 = ld_nt(sp + o0), v1 = ld_nt(sp + o1);
    st_stream(dp, o0, v0);
    st_stream(dp, o1, v1);
    return;
  }
  if (chunks == kThreads) {  // a 4 KiB page (fp8, or bf16 rows of 128 values)
    st_stream(dp, o0, ld_nt(sp + o0));
    return;
  }
  constexpr int U = 4;
  for (int64_t c0 = threadIdx.x; c0 < chunks; c0 += (int64_t)kThreads * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + (int64_t)u * kThreads;
      if (c < chunks) v[u] = ld16(sp + c * 16);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + (int64_t)u * kThreads;
      if (c < chunks) st16(dp + c * 16, v[u]);
    }
  }
}

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int mkv_append_bf16(void* k_pool, void* v_pool, int64_t pool_layer_stride,
                               int64_t num_slots, const void* k_src, const void* v_src,
                               int64_t src_layer_stride, int64_t src_token_stride,
                               const int64_t* slot_mapping, int64_t num_tokens,
                               int32_t num_layers, int32_t row_bytes, int32_t* err,
                               void* stream) {
  clear_error();
  MKV_REQUIRE(num_tokens >= 0 && num_layers >= 0 && num_slots >= 0, MKV_E_INVALID,
              "mkv_append_bf16: negative size");
  if (num_tokens == 0 || num_layers == 0) return MKV_OK;
  MKV_REQUIRE(k_pool && v_pool && k_src && v_src && slot_mapping && err, MKV_E_INVALID,
              "mkv_append_bf16: null pointer");
  MKV_REQUIRE(row_bytes > 0 && row_bytes % 16 == 0, MKV_E_ALIGN,
              "mkv_append_bf16: row_bytes %d is not a positive multiple of 16", row_bytes);
  MKV_REQUIRE(aligned16(k_pool) && aligned16(v_pool) && aligned16(k_src) && aligned16(v_src) &&
                  pool_layer_stride % 16 == 0 && src_layer_stride % 16 == 0 &&
                  src_token_stride % 16 == 0,
              MKV_E_ALIGN, "mkv_append_bf16: pointers and strides must be 16-byte aligned");
  const uint64_t chunks = (uint64_t)num_tokens * (uint64_t)(row_bytes / 16);
  MKV_REQUIRE(chunks < (1ull << 31) && num_layers <= 32767, MKV_E_UNSUPPORTED,
              "mkv_append_bf16: %lld tokens x %d-byte rows x %d layers is too large for one call",
              (long long)num_tokens, row_bytes, num_layers);
  AppendArgs a{(uint8_t*)k_pool, (uint8_t*)v_pool, pool_layer_stride, num_slots,
               (const uint8_t*)k_src, (const uint8_t*)v_src, src_layer_stride, src_token_stride,
               slot_mapping, (uint32_t)num_tokens, (uint32_t)(row_bytes / 16), err};
  dim3 grid((unsigned)((chunks + kThreads - 1) / kThreads), (unsigned)(2 * num_layers));
  if (row_bytes == 512)
    hipLaunchKernelGGL(append_rows_kernel<32>, grid, dim3(kThreads), 0, as_stream(stream), a);
  else
    hipLaunchKernelGGL(append_rows_kernel<0>, grid, dim3(kThreads), 0, as_stream(stream), a);
  return check_launch("mkv_append_bf16");
}

extern "C" int mkv_gather_bf16(const void* k_pool, const void* v_pool, int64_t pool_layer_stride,
                               int64_t num_pages, const int32_t* block_tables,
                               int64_t table_stride, int32_t table_width,
                               const int32_t* seq_lens, const int32_t* starts, int32_t batch,
                               int64_t out_len, const int64_t* out_offsets, void* k_out,
                               void* v_out, int64_t out_layer_stride, int32_t num_layers,
                               int32_t row_bytes, int32_t* err, void* stream) {
  clear_error();
  MKV_REQUIRE(batch >= 0 && out_len >= 0 && num_layers >= 0 && num_pages >= 0 &&
                  table_width >= 0,
              MKV_E_INVALID, "mkv_gather_bf16: negative size");
  if (batch == 0 || out_len == 0 || num_layers == 0) return MKV_OK;
  MKV_REQUIRE(num_layers <= 32767, MKV_E_UNSUPPORTED, "mkv_gather_bf16: too many layers for one call");
  GatherArgs a;
  const int rc = fill_gather_args(a, "mkv_gather_bf16", k_pool, v_pool, pool_layer_stride,
                                  num_pages, block_tables, table_stride, table_width, seq_lens,
                                  starts, batch, out_len, out_offsets, k_out, v_out,
                                  out_layer_stride, row_bytes > 0 ? row_bytes : 1, err);
  if (rc != MKV_OK) return rc;
  hipStream_t s = as_stream(stream);
  switch (row_bytes) {
    case 128: return launch_gather<128>(a, num_layers, s);
    case 256: return launch_gather<256>(a, num_layers, s);
    case 512: return launch_gather<512>(a, num_layers, s);
    case 1024: return launch_gather<1024>(a, num_layers, s);
    case 2048: return launch_gather<2048>(a, num_layers, s);
    default:
      return set_error(MKV_E_UNSUPPORTED,
                       "mkv_gather_bf16: row_bytes %d not in {128,256,512,1024,2048}", row_bytes);
  }
}

extern "C" int mkv_decode_slots(int32_t* seq_lens, int32_t* block_tables, int64_t table_stride,
                                int32_t table_width, const int32_t* new_pages, int32_t batch,
                                int64_t num_pages, int64_t* slot_out, int32_t* err,
                                void* stream) {
  clear_error();
  MKV_REQUIRE(batch >= 0 && table_width >= 0, MKV_E_INVALID, "mkv_decode_slots: negative size");
  if (batch == 0) return MKV_OK;
  MKV_REQUIRE(seq_lens && block_tables && new_pages && slot_out && err, MKV_E_INVALID,
              "mkv_decode_slots: null pointer");
  hipLaunchKernelGGL(decode_slots_kernel, dim3((batch + kThreads - 1) / kThreads),
                     dim3(kThreads), 0, as_stream(stream), seq_lens, block_tables, table_stride,
                     table_width, new_pages, batch, num_pages, slot_out, err);
  return check_launch("mkv_decode_slots");
}

extern "C" int mkv_step_plan(int32_t* block_tables, int64_t table_stride, int32_t table_width,
                             int32_t num_rows, const MkvStepEntry* entries, int32_t num_entries,
                             const int32_t* new_pages, int32_t num_new_pages, int64_t num_pages,
                             int64_t* slot_out, int64_t* pos_out, int64_t num_tokens,
                             int32_t* step_tables, int64_t step_stride, int32_t step_width,
                             int32_t* step_lens, int32_t* rows_out, int64_t* cu_seqlens,
                             int32_t* err, void* stream) {
  clear_error();
  MKV_REQUIRE(num_entries >= 0 && num_rows >= 0 && table_width >= 0 && num_new_pages >= 0 &&
                  num_tokens >= 0 && step_width >= 0 && num_pages >= 0,
              MKV_E_INVALID, "mkv_step_plan: negative size");
  if (num_entries == 0) return MKV_OK;
  MKV_REQUIRE(block_tables && entries && slot_out && pos_out && step_lens && rows_out &&
                  cu_seqlens && err && (new_pages || num_new_pages == 0),
              MKV_E_INVALID, "mkv_step_plan: null pointer");
  MKV_REQUIRE(table_width <= table_stride && (!step_tables || step_width <= step_stride),
              MKV_E_INVALID, "mkv_step_plan: table width exceeds its row stride");
  MKV_REQUIRE(aligned4(entries), MKV_E_ALIGN, "mkv_step_plan: entries must be 4-byte aligned");
  MKV_REQUIRE(num_tokens < ((int64_t)1 << 31), MKV_E_UNSUPPORTED,
              "mkv_step_plan: more than 2^31-1 tokens in one step");
  StepPlanArgs a{block_tables, table_stride, table_width, num_rows, entries, num_entries,
                 new_pages, num_new_pages, num_pages, slot_out, pos_out, num_tokens,
                 step_tables, step_stride, step_width, step_lens, rows_out, cu_seqlens, err};
  hipLaunchKernelGGL(step_plan_kernel, dim3((unsigned)num_entries), dim3(kThreads), 0,
                     as_stream(stream), a);
  return check_launch("mkv_step_plan");
}

extern "C" int mkv_copy_blocks(void* pool, int64_t plane_stride, int32_t num_planes,
                               int64_t num_pages, int64_t page_bytes, const int32_t* src_pages,
                               const int32_t* dst_pages, int32_t n, int32_t* err, void* stream) {
  clear_error();
  MKV_REQUIRE(n >= 0 && num_planes >= 0 && num_pages >= 0, MKV_E_INVALID,
              "mkv_copy_blocks: negative size");
  if (n == 0 || num_planes == 0) return MKV_OK;
  MKV_REQUIRE(pool && src_pages && dst_pages && err, MKV_E_INVALID,
              "mkv_copy_blocks: null pointer");
  MKV_REQUIRE(aligned16(pool) && plane_stride % 16 == 0 && page_bytes > 0 && page_bytes % 16 == 0,
              MKV_E_ALIGN,
              "mkv_copy_blocks: pool, plane stride and page bytes must be 16-byte aligned");
  MKV_REQUIRE(num_planes <= 65535, MKV_E_UNSUPPORTED, "mkv_copy_blocks: too many planes for one call");
  hipLaunchKernelGGL(copy_pages_kernel, dim3((unsigned)n, (unsigned)num_planes), dim3(kThreads), 0,
                     as_stream(stream), (uint8_t*)pool, plane_stride, num_pages, page_bytes,
                     src_pages, dst_pages, err);
  return check_launch("mkv_copy_blocks");
}
