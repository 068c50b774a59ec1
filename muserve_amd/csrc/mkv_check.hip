// mkv_check.hip — opt-in check that an index list names every index at most
// once (gfx950).
//
// The append, scatter, in-place conv and zero kernels require unique slots: a
// repeated slot has no defined winner (the reference's torch index_put_ has
// none either), and in the fp8 append the codes and the scale of a row can
// come from different tokens. This check is what a caller runs in front of
// such a kernel when it wants a repeat reported instead.
//
// One thread per index sets the index's bit in a caller-owned bitmap with an
// atomic OR; a thread that finds its bit already set flags MKV_DEVERR_DUP. A
// second kernel (stream order: every mark is done) clears the words it
// touched, so the bitmap is zero again after every call and never needs a
// clear of its whole size.
#include "mkv_device.h"

namespace mkv {
namespace {

struct UniqueArgs {
  const uint8_t* ids;
  int64_t n;
  int64_t limit;
  uint32_t* bits;
  int32_t* err;
};

template <typename ID>
__device__ __forceinline__ int64_t unique_id(const UniqueArgs& a, int64_t& i) {
  i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= a.n) return -1;
  return (int64_t)reinterpret_cast<const ID*>(a.ids)[i];
}

// Indices outside [0, limit) are left to the kernel that consumes the list
// (it skips and flags them itself); -1 is the append's "skip this token".
template <typename ID>
__global__ __launch_bounds__(kThreads) void unique_mark_kernel(UniqueArgs a) {
  int64_t i;
  const int64_t id = unique_id<ID>(a, i);
  if (id < 0 || id >= a.limit) return;
  const uint32_t bit = 1u << (id & 31);
  const uint32_t old = atomicOr(a.bits + (id >> 5), bit);
  if (old & bit) raise_err(a.err, MKV_DEVERR_DUP);
}

// Every index of the list set a bit in its word, so zeroing those words
// leaves the whole bitmap zero; two indices of one word both store 0.
template <typename ID>
__global__ __launch_bounds__(kThreads) void unique_clear_kernel(UniqueArgs a) {
  int64_t i;
  const int64_t id = unique_id<ID>(a, i);
  if (id < 0 || id >= a.limit) return;
  a.bits[id >> 5] = 0u;
}

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int mkv_check_unique(const void* ids, int32_t id_bytes, int64_t n, int64_t limit,
                                uint32_t* bitmap, int64_t bitmap_words, int32_t* err,
                                void* stream) {
  clear_error();
  MKV_REQUIRE(n >= 0 && limit >= 0, MKV_E_INVALID, "mkv_check_unique: negative size");
  MKV_REQUIRE(id_bytes == 4 || id_bytes == 8, MKV_E_INVALID,
              "mkv_check_unique: id_bytes %d (4 or 8)", id_bytes);
  if (n == 0 || limit == 0) return MKV_OK;
  MKV_REQUIRE(ids && bitmap && err, MKV_E_INVALID, "mkv_check_unique: null pointer");
  MKV_REQUIRE(bitmap_words >= (limit + 31) / 32, MKV_E_INVALID,
              "mkv_check_unique: bitmap of %lld words, %lld needed", (long long)bitmap_words,
              (long long)((limit + 31) / 32));
  MKV_REQUIRE(((uintptr_t)ids & (uintptr_t)(id_bytes - 1)) == 0 && aligned4(bitmap), MKV_E_ALIGN,
              "mkv_check_unique: misaligned ids or bitmap");
  MKV_REQUIRE(n < (1ll << 31), MKV_E_UNSUPPORTED, "mkv_check_unique: more than 2^31 ids");
  const UniqueArgs a{static_cast<const uint8_t*>(ids), n, limit, bitmap, err};
  const dim3 grid((unsigned)((n + kThreads - 1) / kThreads));
  const hipStream_t s = as_stream(stream);
  if (id_bytes == 8) {
    hipLaunchKernelGGL(unique_mark_kernel<int64_t>, grid, dim3(kThreads), 0, s, a);
    hipLaunchKernelGGL(unique_clear_kernel<int64_t>, grid, dim3(kThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL(unique_mark_kernel<int32_t>, grid, dim3(kThreads), 0, s, a);
    hipLaunchKernelGGL(unique_clear_kernel<int32_t>, grid, dim3(kThreads), 0, s, a);
  }
  return check_launch("mkv_check_unique");
}
