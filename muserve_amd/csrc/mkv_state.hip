// mkv_state.hip — GDN recurrent/conv state slot gather and scatter (gfx950).
//
// A state pool is an array of fixed-size entries (one per request slot): for
// the Qwen3.5 GDN layer of one tensor-parallel rank a recurrent state is
// [8, 128, 128] fp32 = 512 KiB and a conv state [2048, 4] bf16 = 16 KiB. Both
// are moved as raw bytes. One launch serves up to two pools so a layer's
// recurrent and conv states travel together. Work is cut into 16 KiB pieces
// (256 threads x 4 x 16 bytes); a workgroup takes one piece, issuing its four
// loads before its four stores.
#include "mkv_device.h"

namespace mkv {
namespace {

constexpr int kUnroll = 4;
constexpr int64_t kMaxGridWgs = 1 << 22;  // bigger jobs loop inside the grid
constexpr int64_t kPiece = (int64_t)kThreads * 16 * kUnroll;  // 16 KiB

struct StateArgs {
  const uint8_t* pool[2];  // gather: source pools; scatter: destination pools
  uint8_t* dense[2];       // gather: outputs;      scatter: inputs
  int64_t bytes[2];
  int64_t pieces_per_entry[2];
  int64_t pieces0;  // number of pieces that belong to pool 0
  int64_t total_pieces;
  int64_t pool_slots;
  const int32_t* slots;
  int32_t* err;
};

template <bool GATHER>
__global__ __launch_bounds__(kThreads) void state_move_kernel(StateArgs a) {
  for (int64_t w = blockIdx.x; w < a.total_pieces; w += gridDim.x) {
    const int which = w < a.pieces0 ? 0 : 1;
    const int64_t local = which == 0 ? w : w - a.pieces0;
    const int64_t b = local / a.pieces_per_entry[which];
    const int64_t piece = local - b * a.pieces_per_entry[which];
    const int64_t bytes = a.bytes[which];
    const int32_t slot = a.slots[b];
    const bool ok = slot >= 0 && slot < a.pool_slots;
    if (!ok && threadIdx.x == 0 && piece == 0 && which == 0) raise_err(a.err, MKV_DEVERR_STATE_SLOT);
    if (!ok && !GATHER) continue;  // scatter: nothing to write for a bad slot
    uint8_t* pool = const_cast<uint8_t*>(a.pool[which]);
    uint8_t* entry = pool + (ok ? (int64_t)slot * bytes : 0);
    uint8_t* dense = a.dense[which] + b * bytes;
    const int64_t base = piece * kPiece;
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t off = base + ((int64_t)u * kThreads + threadIdx.x) * 16;
      v[u] = u32x4{0u, 0u, 0u, 0u};
      if (off < bytes && (ok || !GATHER)) v[u] = GATHER ? ld_nt(entry + off) : ld_nt(dense + off);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t off = base + ((int64_t)u * kThreads + threadIdx.x) * 16;
      if (off < bytes) {
        if (GATHER)
          st16(dense + off, v[u]);
        else
          st_nt(entry + off, v[u]);
      }
    }
  }
}

template <bool GATHER>
int state_move(const char* fn, const void* pool0, int64_t bytes0, const void* dense0,
               const void* pool1, int64_t bytes1, const void* dense1, int64_t pool_slots,
               const int32_t* slots, int32_t n, int32_t* err, hipStream_t stream) {
  clear_error();
  MKV_REQUIRE(n >= 0 && pool_slots >= 0 && bytes0 >= 0 && bytes1 >= 0, MKV_E_INVALID,
              "%s: negative size", fn);
  if (n == 0) return MKV_OK;
  MKV_REQUIRE(slots && err && pool0 && dense0, MKV_E_INVALID, "%s: null pointer", fn);
  const bool two = pool1 != nullptr;
  MKV_REQUIRE(!two || dense1, MKV_E_INVALID, "%s: pool1 given without its dense buffer", fn);
  MKV_REQUIRE(aligned16(pool0) && aligned16(dense0) && bytes0 % 16 == 0 &&
                  (!two || (aligned16(pool1) && aligned16(dense1) && bytes1 % 16 == 0)),
              MKV_E_ALIGN, "%s: pools, buffers and entry sizes must be 16-byte aligned", fn);
  StateArgs a{};
  a.pool[0] = (const uint8_t*)pool0;
  a.dense[0] = (uint8_t*)dense0;
  a.bytes[0] = bytes0;
  a.pieces_per_entry[0] = (bytes0 + kPiece - 1) / kPiece;
  a.pool[1] = two ? (const uint8_t*)pool1 : (const uint8_t*)pool0;
  a.dense[1] = two ? (uint8_t*)dense1 : (uint8_t*)dense0;
  a.bytes[1] = two ? bytes1 : 0;
  a.pieces_per_entry[1] = two ? (bytes1 + kPiece - 1) / kPiece : 0;
  if (a.pieces_per_entry[0] == 0) a.pieces_per_entry[0] = 1;  // zero-byte entries: no-op pieces
  if (two && a.pieces_per_entry[1] == 0) a.pieces_per_entry[1] = 1;
  a.pieces0 = a.pieces_per_entry[0] * n;
  a.total_pieces = a.pieces0 + a.pieces_per_entry[1] * n;
  a.pool_slots = pool_slots;
  a.slots = slots;
  a.err = err;
  const int64_t wgs = a.total_pieces < kMaxGridWgs ? a.total_pieces : kMaxGridWgs;
  hipLaunchKernelGGL((state_move_kernel<GATHER>), dim3((unsigned)wgs), dim3(kThreads), 0, stream,
                     a);
  return check_launch(fn);
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
