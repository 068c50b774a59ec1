// mkv_probe.hip — access-pattern ceilings on gfx950.
//
// Each probe moves the bytes of one product kernel in the same placement and
// does nothing else, so that kernel's rate can be set against what its access
// pattern allows on the device at hand:
//   * read_pages, a workgroup per page: the K and V planes of a list of pages
//     (8 KiB bf16 or 4 KiB fp8 pages of one KV head), 16-byte loads, every
//     page its own workgroup and many resident. The most reads in flight a
//     random page walk can have.
//   * read_pages, a wave per page: the resident grid's waves walk the list
//     (wave w reads pages w, w + W, ...), each page's planes in 1 KiB load
//     instructions with the next page's loads issued before the current one
//     is consumed. The shape of the decode attention's page stream.
//   * scatter_pages: the fp8 append's bytes without the quantisation: 8 KiB
//     of contiguous source read per workgroup, one 4 KiB page written at a
//     listed page id, for `planes` (layer, K|V) planes per launch.
//   * fill: 16-byte streaming stores (device scope, non-temporal), the
//     padded gather's zero tiles.
// Loads feed an xor that is stored only if it equals a constant, so nothing
// is written but the compiler keeps every load. Page ids outside the pool
// are skipped. No reference counterpart: these are measurement kernels that
// bench.py --workload ceilings runs.
#include "mkv_device.h"

namespace mkv {
namespace {

constexpr uint32_t kSinkMagic = 0x6d6b7670u;  // never the xor of random data in practice
constexpr int kSinkSlots = 1024;              // sink: kSinkSlots 16-byte slots

__device__ __forceinline__ void keep(u32x4 acc, u32x4* sink, uint32_t slot) {
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == kSinkMagic) sink[slot & (kSinkSlots - 1)] = acc;
}

template <bool NT>
__device__ __forceinline__ u32x4 probe_ld(const uint8_t* p) {
  if constexpr (NT) return ld_nt(p);
  else return ld16(p);
}

// A workgroup per page: page pages[blockIdx.x]'s K and V planes, PB bytes
// each, 16 bytes a thread per 4 KiB step.
template <int PB, bool NT>
__global__ __launch_bounds__(kThreads) void probe_read_wg_kernel(const uint8_t* kp, const uint8_t* vp,
                                                                 const int32_t* pages, int64_t num_pages,
                                                                 u32x4* sink) {
  const int64_t pg = ld_const(pages + blockIdx.x);
  if (pg < 0 || pg >= num_pages) return;
  u32x4 acc = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < PB / 4096; ++i) {
    acc ^= probe_ld<NT>(kp + pg * PB + i * 4096 + threadIdx.x * 16);
    acc ^= probe_ld<NT>(vp + pg * PB + i * 4096 + threadIdx.x * 16);
  }
  keep(acc, sink, blockIdx.x);
}

// A wave per page over the resident grid: wave w reads pages w, w + W, ...
// (W waves), a page's two planes in PB / 1024 load instructions each, the
// next page's loads issued before the current page is consumed.
template <int PB, bool NT>
__global__ __launch_bounds__(kThreads) void probe_read_walk_kernel(const uint8_t* kp, const uint8_t* vp,
                                                                   const int32_t* pages, int64_t n,
                                                                   int64_t num_pages, u32x4* sink) {
  constexpr int L = PB / 1024;  // load instructions per plane
  const int lane = threadIdx.x & 63;
  const int64_t w0 = (int64_t)blockIdx.x * (kThreads / 64) + threadIdx.x / 64;
  const int64_t stride = (int64_t)gridDim.x * (kThreads / 64);
  auto load = [&](u32x4 (&buf)[2 * L], int64_t p) __attribute__((always_inline)) {
    int64_t pg = p < n ? (int64_t)pages[p] : -1;
    if (pg >= num_pages) pg = -1;
#pragma unroll
    for (int i = 0; i < L; ++i) {
      if (pg >= 0) {
        buf[i] = probe_ld<NT>(kp + pg * PB + i * 1024 + lane * 16);
        buf[L + i] = probe_ld<NT>(vp + pg * PB + i * 1024 + lane * 16);
      } else {
        buf[i] = buf[L + i] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  u32x4 acc = {0u, 0u, 0u, 0u};
  u32x4 cur[2 * L], nxt[2 * L];
  load(cur, w0);
  for (int64_t p = w0; p < n; p += stride) {
    load(nxt, p + stride);
#pragma unroll
    for (int i = 0; i < 2 * L; ++i) {
      acc ^= cur[i];
      cur[i] = nxt[i];
    }
  }
  keep(acc, sink, (uint32_t)w0);
}

// Workgroup (x, y): 8 KiB of plane y's source at x * 8192 (two 16-byte
// non-temporal loads a thread), xor-folded to 4 KiB and stored to plane y's
// page pages[x] (one 16-byte non-temporal store a thread).
__global__ __launch_bounds__(kThreads) void probe_scatter_kernel(const uint8_t* src, int64_t src_plane,
                                                                 uint8_t* dst, int64_t dst_plane,
                                                                 int64_t dst_pages, const int32_t* pages) {
  const int64_t pg = ld_const(pages + blockIdx.x);
  if (pg < 0 || pg >= dst_pages) return;
  const uint8_t* s = src + blockIdx.y * src_plane + (int64_t)blockIdx.x * 8192 + threadIdx.x * 32;
  const u32x4 a = ld_nt(s), b = ld_nt(s + 16);
  st_nt(dst + blockIdx.y * dst_plane + pg * 4096 + threadIdx.x * 16, a ^ b);
}

// One 16-byte streaming store of zeros a thread, 4 KiB a workgroup.
__global__ __launch_bounds__(kThreads) void probe_fill_kernel(uint8_t* dst) {
  st_stream(dst + (int64_t)blockIdx.x * 4096, threadIdx.x * 16, u32x4{0u, 0u, 0u, 0u});
}

int resident_grid(const void* kernel) {
  int dev = 0, cus = 0, per = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, kThreads, 0) != hipSuccess)
    return -1;
  return cus * per;
}

template <int PB, bool NT>
int launch_read(const uint8_t* kp, const uint8_t* vp, int64_t num_pages, const int32_t* pages,
                int64_t n, int walk, u32x4* sink, hipStream_t st) {
  if (!walk) {
    hipLaunchKernelGGL((probe_read_wg_kernel<PB, NT>), dim3((unsigned)n), dim3(kThreads), 0, st, kp,
                       vp, pages, num_pages, sink);
  } else {
    const int grid = resident_grid(reinterpret_cast<const void*>(probe_read_walk_kernel<PB, NT>));
    MKV_REQUIRE(grid > 0, MKV_E_LAUNCH, "mkv_probe_read_pages: no resident grid");
    hipLaunchKernelGGL((probe_read_walk_kernel<PB, NT>), dim3((unsigned)grid), dim3(kThreads), 0, st,
                       kp, vp, pages, n, num_pages, sink);
  }
  return check_launch("mkv_probe_read_pages");
}

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int mkv_probe_read_pages(const void* k_planes, const void* v_planes, int32_t page_bytes,
                                    int64_t num_pages, const int32_t* pages, int64_t n,
                                    int32_t walk, int32_t nontemporal, void* sink, void* stream) {
  clear_error();
  MKV_REQUIRE(page_bytes == 4096 || page_bytes == 8192, MKV_E_UNSUPPORTED,
              "mkv_probe_read_pages: page_bytes must be 4096 or 8192, got %d", (int)page_bytes);
  MKV_REQUIRE(n >= 0 && num_pages >= 0, MKV_E_INVALID, "mkv_probe_read_pages: negative size");
  MKV_REQUIRE(n <= 0x7fffffff, MKV_E_UNSUPPORTED, "mkv_probe_read_pages: more than 2^31-1 pages");
  if (n == 0) return MKV_OK;
  MKV_REQUIRE(k_planes && v_planes && pages && sink, MKV_E_INVALID, "mkv_probe_read_pages: null pointer");
  MKV_REQUIRE(aligned16(k_planes) && aligned16(v_planes) && aligned16(sink), MKV_E_ALIGN,
              "mkv_probe_read_pages: planes and sink must be 16-byte aligned");
  const auto* kp = static_cast<const uint8_t*>(k_planes);
  const auto* vp = static_cast<const uint8_t*>(v_planes);
  auto* sk = static_cast<u32x4*>(sink);
  const hipStream_t st = as_stream(stream);
  if (page_bytes == 8192)
    return nontemporal ? launch_read<8192, true>(kp, vp, num_pages, pages, n, walk, sk, st)
                       : launch_read<8192, false>(kp, vp, num_pages, pages, n, walk, sk, st);
  return nontemporal ? launch_read<4096, true>(kp, vp, num_pages, pages, n, walk, sk, st)
                     : launch_read<4096, false>(kp, vp, num_pages, pages, n, walk, sk, st);
}

extern "C" int mkv_probe_scatter_pages(const void* src, int64_t src_plane, void* dst, int64_t dst_plane,
                                       int64_t dst_pages, const int32_t* pages, int32_t npages,
                                       int32_t planes, void* stream) {
  clear_error();
  MKV_REQUIRE(npages >= 0 && planes >= 0 && dst_pages >= 0, MKV_E_INVALID,
              "mkv_probe_scatter_pages: negative size");
  MKV_REQUIRE(planes <= 65535, MKV_E_UNSUPPORTED, "mkv_probe_scatter_pages: more than 65535 planes");
  if (npages == 0 || planes == 0) return MKV_OK;
  MKV_REQUIRE(src && dst && pages, MKV_E_INVALID, "mkv_probe_scatter_pages: null pointer");
  MKV_REQUIRE(aligned16(src) && aligned16(dst) && src_plane % 16 == 0 && dst_plane % 16 == 0,
              MKV_E_ALIGN, "mkv_probe_scatter_pages: buffers and plane strides must be 16-byte aligned");
  MKV_REQUIRE(src_plane >= (int64_t)npages * 8192 && dst_plane >= dst_pages * 4096, MKV_E_INVALID,
              "mkv_probe_scatter_pages: a plane is shorter than its pages");
  hipLaunchKernelGGL(probe_scatter_kernel, dim3((unsigned)npages, (unsigned)planes), dim3(kThreads), 0,
                     as_stream(stream), static_cast<const uint8_t*>(src), src_plane,
                     static_cast<uint8_t*>(dst), dst_plane, dst_pages, pages);
  return check_launch("mkv_probe_scatter_pages");
}

extern "C" int mkv_probe_fill(void* dst, int64_t bytes, void* stream) {
  clear_error();
  MKV_REQUIRE(bytes >= 0 && bytes % 4096 == 0, MKV_E_INVALID,
              "mkv_probe_fill: bytes must be a non-negative multiple of 4096");
  MKV_REQUIRE(bytes / 4096 <= 0x7fffffff, MKV_E_UNSUPPORTED, "mkv_probe_fill: more than 2^31-1 tiles");
  if (bytes == 0) return MKV_OK;
  MKV_REQUIRE(dst && aligned16(dst), MKV_E_ALIGN, "mkv_probe_fill: dst must be 16-byte aligned");
  hipLaunchKernelGGL(probe_fill_kernel, dim3((unsigned)(bytes / 4096)), dim3(kThreads), 0,
                     as_stream(stream), static_cast<uint8_t*>(dst));
  return check_launch("mkv_probe_fill");
}
