// mkv_state.hip — GDN recurrent/conv state slot gather and scatter, and the
// layered block pack / unpack of the host tier (gfx950).
//
// A state pool is an array of fixed-size entries (one per request slot): for
// the Qwen3.5 GDN layer of one tensor-parallel rank a recurrent state is
// [8, 128, 128] fp32 = 512 KiB and a conv state [2048, 4] bf16 = 16 KiB. Both
// are moved as raw bytes. One launch serves up to two pools so a layer's
// recurrent and conv states travel together. Work is cut into 16 KiB pieces
// (256 threads x 4 x 16 bytes): grid.x is the piece within an entry (pool 0's
// pieces, then pool 1's), grid.y the entry, so nothing is decoded by
// division; a workgroup issues its four loads before its four stores. Loads
// are non-temporal; a gather's output uses ordinary stores (the layer that
// gathered it reads it next, often still from the MALL), a scatter's pool
// writes streaming ones (st_stream: the slot is not read again this step).
//
// grid.z is the plane of a layered pool (a KV pool's [layer, K|V] planes, a
// state pool's layers): plane z's entries start at pool + z * plane_stride and
// its dense rows at dense + z * n * entry_bytes. Pack / unpack move the blocks
// of every plane between the pool and one contiguous buffer, which may be
// pinned host memory: the kernel's loads or stores then cross the host link
// directly (no staging copy), at the link's rate.
#include "mkv_device.h"

namespace mkv {
namespace {

constexpr int kUnroll = 4;
constexpr int64_t kPiece = (int64_t)kThreads * 16 * kUnroll;  // 16 KiB
constexpr unsigned kMaxGridY = 65535;                          // more entries loop in the grid

struct StateArgs {
  const uint8_t* pool0;  // gather: source pools; scatter: destination pools
  const uint8_t* pool1;
  uint8_t* dense0;       // gather: outputs;      scatter: inputs
  uint8_t* dense1;
  int64_t bytes0, bytes1;
  uint32_t pieces0;  // pieces per pool-0 entry (grid.x below it is pool 0)
  int64_t plane_stride;  // bytes between planes of pool 0 (grid.z); 0 with one plane
  int64_t pool_slots;
  const int32_t* slots;
  int32_t n;
  int32_t* err;
};

// base is the workgroup's piece (uniform), off the lane's offset in it
template <bool GATHER>
__device__ __forceinline__ void store(uint8_t* base, uint32_t off, u32x4 v) {
  if (GATHER)
    st16(base + off, v);
  else
    st_stream(base, off, v);
}

// One workgroup's piece `bx` (grid.x) of every entry it covers.
template <bool GATHER>
__device__ __forceinline__ void move_piece(const StateArgs& a, uint32_t bx) {
  const bool second = bx >= a.pieces0;
  const int64_t piece = second ? bx - a.pieces0 : bx;
  const int64_t bytes = second ? a.bytes1 : a.bytes0;
  const uint8_t* pool = second ? a.pool1 : a.pool0;
  uint8_t* dense = second ? a.dense1 : a.dense0;
  const int64_t base = piece * kPiece;
  const bool full = base + kPiece <= bytes;
  const int64_t plane = blockIdx.z;  // pool 1 has one plane
  pool += plane * a.plane_stride;
  dense += plane * a.n * bytes;
  for (int64_t b = blockIdx.y; b < a.n; b += gridDim.y) {
    const int32_t slot = ld_const(a.slots + b);
    uint8_t* row = dense + b * bytes + base;
    u32x4 v[kUnroll];
    if (!GATHER && full) {
      // scatter: the dense row does not depend on the slot, so it is loaded
      // with the slot's (scalar) load; the empty asm keeps the compiler from
      // moving these loads behind the slot check: one round trip, not two
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = ld_nt(row + (u * kThreads + threadIdx.x) * 16);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) asm volatile("" : "+v"(v[u]));
    }
    const bool ok = slot >= 0 && slot < a.pool_slots;
    if (!ok && threadIdx.x == 0 && piece == 0 && !second && plane == 0)
      raise_err(a.err, MKV_DEVERR_STATE_SLOT);
    if (!ok && !GATHER) continue;  // scatter: nothing to write for a bad slot
    uint8_t* entry = const_cast<uint8_t*>(pool) + (ok ? (int64_t)slot * bytes : 0) + base;
    const uint8_t* src = GATHER ? entry : row;
    uint8_t* dst = GATHER ? row : entry;
    if (!GATHER && full) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) store<GATHER>(dst, (u * kThreads + threadIdx.x) * 16, v[u]);
      continue;
    }
    if (full && ok) {  // straight-line: every load issued before any store
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = ld_nt(src + (u * kThreads + threadIdx.x) * 16);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) store<GATHER>(dst, (u * kThreads + threadIdx.x) * 16, v[u]);
      continue;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {  // an entry's last piece, or a bad slot (zeros)
      const int64_t off = (u * kThreads + threadIdx.x) * 16;
      v[u] = u32x4{0u, 0u, 0u, 0u};
      if (ok && base + off < bytes) v[u] = ld_nt(src + off);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t off = (u * kThreads + threadIdx.x) * 16;
      if (base + off < bytes) store<GATHER>(dst, (uint32_t)off, v[u]);
    }
  }
}

template <bool GATHER>
__global__ __launch_bounds__(kThreads) void state_move_kernel(StateArgs a) {
  move_piece<GATHER>(a, blockIdx.x);
}

constexpr int kEmpty = 1;  // argument check passed, nothing to launch

// Checks a move's arguments and fills `a`; `pieces` = grid.x.
int state_args(const char* fn, const void* pool0, int64_t bytes0, const void* dense0,
               const void* pool1, int64_t bytes1, const void* dense1, int64_t pool_slots,
               const int32_t* slots, int32_t n, int32_t* err, int32_t planes,
               int64_t plane_stride, StateArgs& a, int64_t& pieces) {
  MKV_REQUIRE(n >= 0 && pool_slots >= 0 && bytes0 >= 0 && bytes1 >= 0 && planes >= 1 &&
                  plane_stride >= 0,
              MKV_E_INVALID, "%s: negative size", fn);
  MKV_REQUIRE(planes == 1 || (pool1 == nullptr && plane_stride % 16 == 0 &&
                              plane_stride >= pool_slots * bytes0),
              MKV_E_INVALID, "%s: planes must not overlap (plane_stride >= blocks x bytes)", fn);
  MKV_REQUIRE(planes <= (int32_t)kMaxGridY, MKV_E_UNSUPPORTED, "%s: more than %u planes", fn,
              kMaxGridY);
  if (n == 0) return kEmpty;
  MKV_REQUIRE(slots && err && pool0 && dense0, MKV_E_INVALID, "%s: null pointer", fn);
  const bool two = pool1 != nullptr;
  MKV_REQUIRE(!two || dense1, MKV_E_INVALID, "%s: pool1 given without its dense buffer", fn);
  MKV_REQUIRE(aligned16(pool0) && aligned16(dense0) && bytes0 % 16 == 0 &&
                  (!two || (aligned16(pool1) && aligned16(dense1) && bytes1 % 16 == 0)),
              MKV_E_ALIGN, "%s: pools, buffers and entry sizes must be 16-byte aligned", fn);
  // a zero-byte entry still gets one (empty) piece: it reports bad slots
  const int64_t p0 = bytes0 > 0 ? (bytes0 + kPiece - 1) / kPiece : 1;
  const int64_t p1 = two ? (bytes1 > 0 ? (bytes1 + kPiece - 1) / kPiece : 1) : 0;
  MKV_REQUIRE(p0 + p1 < (1ll << 31), MKV_E_UNSUPPORTED, "%s: entries too large", fn);
  a.pool0 = (const uint8_t*)pool0;
  a.dense0 = (uint8_t*)dense0;
  a.bytes0 = bytes0;
  a.pool1 = two ? (const uint8_t*)pool1 : (const uint8_t*)pool0;
  a.dense1 = two ? (uint8_t*)dense1 : (uint8_t*)dense0;
  a.bytes1 = two ? bytes1 : 0;
  a.pieces0 = (uint32_t)p0;
  a.plane_stride = plane_stride;
  a.pool_slots = pool_slots;
  a.slots = slots;
  a.n = n;
  a.err = err;
  pieces = p0 + p1;
  return MKV_OK;
}

template <bool GATHER>
int state_move(const char* fn, const void* pool0, int64_t bytes0, const void* dense0,
               const void* pool1, int64_t bytes1, const void* dense1, int64_t pool_slots,
               const int32_t* slots, int32_t n, int32_t* err, hipStream_t stream,
               int32_t planes = 1, int64_t plane_stride = 0) {
  clear_error();
  StateArgs a{};
  int64_t pieces = 0;
  const int rc = state_args(fn, pool0, bytes0, dense0, pool1, bytes1, dense1, pool_slots, slots,
                            n, err, planes, plane_stride, a, pieces);
  if (rc != MKV_OK) return rc == kEmpty ? MKV_OK : rc;
  const dim3 grid((unsigned)pieces, (unsigned)n < kMaxGridY ? (unsigned)n : kMaxGridY,
                  (unsigned)planes);
  hipLaunchKernelGGL((state_move_kernel<GATHER>), grid, dim3(kThreads), 0, stream, a);
  return check_launch(fn);
}

// ---------------------------------------------------------------------------
// Block zero-fill of a layered pool: a new request's GDN state slots start as
// zeros in every layer. Same grid as the moves (piece, block, plane); every
// store is a streaming zero store.
// ---------------------------------------------------------------------------
struct ZeroArgs {
  uint8_t* pool;
  int64_t bytes;
  int64_t plane_stride;
  int64_t pool_blocks;
  const int32_t* ids;
  int32_t n;
  int32_t* err;
};

__global__ __launch_bounds__(kThreads) void zero_blocks_kernel(ZeroArgs a) {
  const int64_t base = (int64_t)blockIdx.x * kPiece;
  uint8_t* plane = a.pool + (int64_t)blockIdx.z * a.plane_stride;
  for (int64_t b = blockIdx.y; b < a.n; b += gridDim.y) {
    const int32_t id = a.ids[b];
    if (id < 0 || id >= a.pool_blocks) {
      if (threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.z == 0)
        raise_err(a.err, MKV_DEVERR_STATE_SLOT);
      continue;
    }
    uint8_t* blk = plane + (int64_t)id * a.bytes + base;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t off = (u * kThreads + threadIdx.x) * 16;
      if (base + off < a.bytes) st_stream(blk, (uint32_t)off, u32x4{0u, 0u, 0u, 0u});
    }
  }
}

// ---------------------------------------------------------------------------
// GDN decode conv (muserve/model/qwen35_layer_v2.py:163-201, decode branch
// :187-192), per request slot and in place:
//   out[b,c] = silu(sum_k w[c,k] p_k), p = (state[c, W-3 .. W-1], x[b,c]),
//   state[c] <- (state[c, 1 .. W-1], x[b,c]),
// fp32 arithmetic, bf16 in and out. A slot holds the last W (3 or 4) inputs of
// each channel, oldest first, [C, W] bf16; the kernel width is 4. The slot is
// read once and written once per step: no dense gather / scatter of the conv
// state. A thread takes 8 channels (16-byte loads of x, out and the weights,
// W 16-byte loads of the state); grid = (channel groups / 256, batch).
// ---------------------------------------------------------------------------
constexpr int kConvK = 4;

struct ConvArgs {
  uint8_t* pool;         // [pool_slots, C, W] bf16
  const uint8_t* x;      // [B, C] bf16
  const uint8_t* w;      // [C, 4] bf16
  uint8_t* out;          // [B, C] bf16
  const int32_t* slots;  // [B], unique
  int64_t pool_slots;
  int32_t channels, batch;
  int32_t* err;
};

__device__ __forceinline__ uint32_t half16(const u32x4* v, int e) {  // bf16 element e
  const uint32_t w = v[e >> 3][(e >> 1) & 3];
  return (e & 1) ? (w >> 16) : (w & 0xffffu);
}

// Channel groups of workgroup `bx` for request b.
template <int W>
__device__ __forceinline__ void conv_row(const ConvArgs& a, uint32_t bx, int64_t b) {
  static_assert(W >= kConvK - 1 && W <= 4, "conv state width");
  const int32_t g = bx * kThreads + threadIdx.x;  // group of 8 channels
  if (g * 8 >= a.channels) return;
  const int32_t slot = a.slots[b];
  uint8_t* outp = a.out + (b * a.channels + g * 8) * 2;
  if (slot < 0 || slot >= a.pool_slots) {  // nothing to convolve: zeros, the pool untouched
    if (g == 0) raise_err(a.err, MKV_DEVERR_STATE_SLOT);
    st16(outp, u32x4{0u, 0u, 0u, 0u});
    return;
  }
  uint8_t* st = a.pool + ((int64_t)slot * a.channels + g * 8) * (W * 2);
  u32x4 sv[W], wv[kConvK];
#pragma unroll
  for (int j = 0; j < W; ++j) sv[j] = ld16(st + 16 * j);
  const u32x4 xv = ld16(a.x + (b * a.channels + g * 8) * 2);
#pragma unroll
  for (int j = 0; j < kConvK; ++j) wv[j] = ld16(a.w + ((int64_t)g * 8 * kConvK) * 2 + 16 * j);
  uint32_t outw[4] = {0u, 0u, 0u, 0u};
  uint32_t nsw[4 * W];
#pragma unroll
  for (int j = 0; j < 4 * W; ++j) nsw[j] = 0u;
#pragma unroll
  for (int ch = 0; ch < 8; ++ch) {
    const uint32_t xb = half16(&xv, ch);
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < kConvK; ++k) {
      const uint32_t pb = k < kConvK - 1 ? half16(sv, ch * W + (W - (kConvK - 1)) + k) : xb;
      acc = fmaf(bits_f32(half16(wv, ch * kConvK + k) << 16), bits_f32(pb << 16), acc);
    }
    const float y = acc / (1.0f + expf(-acc));
    outw[ch >> 1] |= (uint32_t)f32_to_bf16_rne(y) << (16 * (ch & 1));
#pragma unroll
    for (int j = 0; j < W; ++j) {  // shifted state: inputs 1 .. W-1, then x
      const uint32_t v = j < W - 1 ? half16(sv, ch * W + j + 1) : xb;
      const int e = ch * W + j;
      nsw[e >> 1] |= v << (16 * (e & 1));
    }
  }
  st16(outp, u32x4{outw[0], outw[1], outw[2], outw[3]});
#pragma unroll
  for (int j = 0; j < W; ++j)
    st16(st + 16 * j, u32x4{nsw[4 * j], nsw[4 * j + 1], nsw[4 * j + 2], nsw[4 * j + 3]});
}

template <int W>
__global__ __launch_bounds__(kThreads) void conv_decode_kernel(ConvArgs a) {
  conv_row<W>(a, blockIdx.x, blockIdx.y);
}

// The decode step's state reads of one GDN layer in one launch: workgroups
// below s.pieces0 gather the batch's recurrent states (move_piece), the rest
// run the conv in place on the conv slots (conv_row); grid.y is the request.
template <int W>
__global__ __launch_bounds__(kThreads) void gdn_decode_gather_kernel(StateArgs s, ConvArgs c) {
  if (blockIdx.x < s.pieces0)
    move_piece<true>(s, blockIdx.x);
  else
    conv_row<W>(c, blockIdx.x - s.pieces0, blockIdx.y);
}

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int mkv_state_gather(const void* pool0, int64_t entry_bytes0, void* out0,
                                const void* pool1, int64_t entry_bytes1, void* out1,
                                int64_t pool_slots, const int32_t* slots, int32_t n, int32_t* err,
                                void* stream) {
  return state_move<true>("mkv_state_gather", pool0, entry_bytes0, out0, pool1, entry_bytes1,
                          out1, pool_slots, slots, n, err, as_stream(stream));
}

extern "C" int mkv_state_scatter(void* pool0, int64_t entry_bytes0, const void* in0, void* pool1,
                                 int64_t entry_bytes1, const void* in1, int64_t pool_slots,
                                 const int32_t* slots, int32_t n, int32_t* err, void* stream) {
  return state_move<false>("mkv_state_scatter", pool0, entry_bytes0, in0, pool1, entry_bytes1,
                           in1, pool_slots, slots, n, err, as_stream(stream));
}

extern "C" int mkv_pack_blocks(const void* pool, int64_t plane_stride, int32_t num_planes,
                               int64_t block_bytes, int64_t pool_blocks, const int32_t* ids,
                               int32_t n, void* out, int32_t* err, void* stream) {
  return state_move<true>("mkv_pack_blocks", pool, block_bytes, out, nullptr, 0, nullptr,
                          pool_blocks, ids, n, err, as_stream(stream), num_planes,
                          num_planes > 1 ? plane_stride : 0);
}

extern "C" int mkv_unpack_blocks(void* pool, int64_t plane_stride, int32_t num_planes,
                                 int64_t block_bytes, int64_t pool_blocks, const int32_t* ids,
                                 int32_t n, const void* in, int32_t* err, void* stream) {
  return state_move<false>("mkv_unpack_blocks", pool, block_bytes, in, nullptr, 0, nullptr,
                           pool_blocks, ids, n, err, as_stream(stream), num_planes,
                           num_planes > 1 ? plane_stride : 0);
}

extern "C" int mkv_zero_blocks(void* pool, int64_t plane_stride, int32_t num_planes,
                               int64_t block_bytes, int64_t pool_blocks, const int32_t* ids,
                               int32_t n, int32_t* err, void* stream) {
  clear_error();
  MKV_REQUIRE(n >= 0 && pool_blocks >= 0 && block_bytes >= 0 && plane_stride >= 0 &&
                  num_planes >= 1,
              MKV_E_INVALID, "mkv_zero_blocks: negative size");
  MKV_REQUIRE(num_planes <= (int32_t)kMaxGridY, MKV_E_UNSUPPORTED,
              "mkv_zero_blocks: more than %u planes", kMaxGridY);
  MKV_REQUIRE(num_planes == 1 || plane_stride >= pool_blocks * block_bytes, MKV_E_INVALID,
              "mkv_zero_blocks: planes must not overlap (plane_stride >= blocks x bytes)");
  if (n == 0 || block_bytes == 0) return MKV_OK;
  MKV_REQUIRE(pool && ids && err, MKV_E_INVALID, "mkv_zero_blocks: null pointer");
  MKV_REQUIRE(aligned16(pool) && block_bytes % 16 == 0 &&
                  (num_planes == 1 || plane_stride % 16 == 0),
              MKV_E_ALIGN, "mkv_zero_blocks: pool, block bytes and plane stride must be 16-byte aligned");
  const int64_t pieces = (block_bytes + kPiece - 1) / kPiece;
  MKV_REQUIRE(pieces < (1ll << 31), MKV_E_UNSUPPORTED, "mkv_zero_blocks: blocks too large");
  ZeroArgs a{(uint8_t*)pool, block_bytes, num_planes > 1 ? plane_stride : 0, pool_blocks, ids, n,
             err};
  const dim3 grid((unsigned)pieces, (unsigned)n < kMaxGridY ? (unsigned)n : kMaxGridY,
                  (unsigned)num_planes);
  hipLaunchKernelGGL(zero_blocks_kernel, grid, dim3(kThreads), 0, as_stream(stream), a);
  return check_launch("mkv_zero_blocks");
}

namespace mkv {
namespace {

// Checks a decode conv's arguments and fills `a`.
int conv_args(const char* fn, void* conv_pool, int64_t pool_slots, int32_t channels,
              int32_t width, const int32_t* slots, int32_t batch, const void* x,
              const void* weight, int32_t kernel_size, void* out, int32_t* err, ConvArgs& a) {
  MKV_REQUIRE(pool_slots >= 0 && channels > 0 && batch >= 0, MKV_E_INVALID, "%s: bad sizes", fn);
  MKV_REQUIRE(kernel_size == kConvK && (width == 3 || width == 4), MKV_E_UNSUPPORTED,
              "%s: kernel %d / state width %d unsupported (kernel 4, width 3 or 4)", fn,
              kernel_size, width);
  MKV_REQUIRE(channels % 8 == 0, MKV_E_UNSUPPORTED, "%s: channels must be a multiple of 8", fn);
  if (batch == 0) return kEmpty;
  MKV_REQUIRE(conv_pool && slots && x && weight && out && err, MKV_E_INVALID, "%s: null pointer",
              fn);
  MKV_REQUIRE(aligned16(conv_pool) && aligned16(x) && aligned16(weight) && aligned16(out),
              MKV_E_ALIGN, "%s: pool, x, weight and out must be 16-byte aligned", fn);
  MKV_REQUIRE(batch <= 65535, MKV_E_UNSUPPORTED, "%s: batch above 65535", fn);
  a.pool = static_cast<uint8_t*>(conv_pool);
  a.x = static_cast<const uint8_t*>(x);
  a.w = static_cast<const uint8_t*>(weight);
  a.out = static_cast<uint8_t*>(out);
  a.slots = slots;
  a.pool_slots = pool_slots;
  a.channels = channels;
  a.batch = batch;
  a.err = err;
  return MKV_OK;
}

int64_t conv_groups(int32_t channels) { return (channels / 8 + kThreads - 1) / kThreads; }

}  // namespace
}  // namespace mkv

extern "C" int mkv_gdn_conv_decode(void* conv_pool, int64_t pool_slots, int32_t channels,
                                   int32_t width, const int32_t* slots, int32_t batch,
                                   const void* x, const void* weight, int32_t kernel_size,
                                   void* out, int32_t* err, void* stream) {
  clear_error();
  const char* fn = "mkv_gdn_conv_decode";
  ConvArgs a{};
  const int rc = conv_args(fn, conv_pool, pool_slots, channels, width, slots, batch, x, weight,
                           kernel_size, out, err, a);
  if (rc != MKV_OK) return rc == kEmpty ? MKV_OK : rc;
  const dim3 grid((unsigned)conv_groups(channels), (unsigned)batch);
  if (width == 3)
    hipLaunchKernelGGL(conv_decode_kernel<3>, grid, dim3(kThreads), 0, as_stream(stream), a);
  else
    hipLaunchKernelGGL(conv_decode_kernel<4>, grid, dim3(kThreads), 0, as_stream(stream), a);
  return check_launch(fn);
}

extern "C" int mkv_gdn_decode_gather(const void* state_pool, int64_t state_bytes,
                                     void* state_out, void* conv_pool, int32_t channels,
                                     int32_t width, int64_t pool_slots, const int32_t* slots,
                                     int32_t batch, const void* x, const void* weight,
                                     int32_t kernel_size, void* conv_out, int32_t* err,
                                     void* stream) {
  clear_error();
  const char* fn = "mkv_gdn_decode_gather";
  StateArgs s{};
  int64_t pieces = 0;
  const int rs = state_args(fn, state_pool, state_bytes, state_out, nullptr, 0, nullptr,
                            pool_slots, slots, batch, err, 1, 0, s, pieces);
  if (rs < 0) return rs;
  ConvArgs c{};
  const int rc = conv_args(fn, conv_pool, pool_slots, channels, width, slots, batch, x, weight,
                           kernel_size, conv_out, err, c);
  if (rc < 0) return rc;
  if (rs == kEmpty || rc == kEmpty) return MKV_OK;  // batch 0
  const dim3 grid((unsigned)(pieces + conv_groups(channels)), (unsigned)batch);
  if (width == 3)
    hipLaunchKernelGGL(gdn_decode_gather_kernel<3>, grid, dim3(kThreads), 0, as_stream(stream), s,
                       c);
  else
    hipLaunchKernelGGL(gdn_decode_gather_kernel<4>, grid, dim3(kThreads), 0, as_stream(stream), s,
                       c);
  return check_launch(fn);
}
