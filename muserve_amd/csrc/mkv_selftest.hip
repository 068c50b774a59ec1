// mkv_selftest.hip — on-device check of the conversions the fp8 kernels rely
// on, with the exact builtins and compiler flags they are built with.
//
// Compares, over every fp32 bit pattern, gfx950's v_cvt_pk_fp8_f32 (both
// halves) with the integer RNE encoder of mkv_common.h (which equals torch's
// CPU cast on all 2^32 inputs) for |x| <= 448 and NaN, and v_cvt_pk_bf16_f32
// with round-to-nearest-even bf16; v_cvt_pk_f32_fp8 (both halves) with the
// OCP decode of all 256 codes, and v_cvt_scalef32_pk_bf16_fp8 at scale 1
// (both halves) with the bf16 of that decode; and div_by_recip with IEEE
// division over the fp8 quantiser's whole domain (every non-negative bf16 absmax pattern,
// inf and NaN included, as divisor source; every bf16 x with |x| <= absmax,
// or every x for a NaN absmax; NaN codes compare equal). Runs in a few
// milliseconds.
#include "mkv_device.h"

namespace mkv {
namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

enum { kFp8, kBf16, kDecode, kDivCode, kDivQuot, kValues, kPairs, kCounters };

__device__ __forceinline__ bool bf16_is_nan(uint32_t h) {
  return (h & 0x7f80u) == 0x7f80u && (h & 0x7fu) != 0;
}
__device__ __forceinline__ float clamp448(float x) {
  return x < -448.0f ? -448.0f : (x > 448.0f ? 448.0f : x);
}

__global__ __launch_bounds__(256) void check_conversions_kernel(unsigned long long* out) {
  __shared__ unsigned long long acc[kCounters];
  if (threadIdx.x < kCounters) acc[threadIdx.x] = 0;
  __syncthreads();
  unsigned long long c[kCounters] = {0, 0, 0, 0, 0, 0, 0};
  const unsigned long long stride = (unsigned long long)gridDim.x * blockDim.x;
  const unsigned long long first = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x;
  for (unsigned long long u = first; u < (1ull << 32); u += stride) {
    const float x = bits_f32((uint32_t)u);
    const bool nan = x != x;
    const float y = bits_f32((uint32_t)u ^ 0x80000000u);  // the same value negated
    const uint32_t pk = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(
        x, y, __builtin_amdgcn_cvt_pk_fp8_f32(y, x, 0, false), true);
    if (nan) {
      c[kFp8] += ((pk & 0x7fu) != 0x7fu) + (((pk >> 8) & 0x7fu) != 0x7fu) +
                 (((pk >> 16) & 0x7fu) != 0x7fu) + (((pk >> 24) & 0x7fu) != 0x7fu);
    } else if (x >= -448.0f && x <= 448.0f) {
      const uint32_t ex = f32_to_e4m3fn(x), ey = f32_to_e4m3fn(y);
      c[kFp8] += ((pk & 0xffu) != ey) + (((pk >> 8) & 0xffu) != ex) +
                 (((pk >> 16) & 0xffu) != ex) + ((pk >> 24) != ey);
    }
    const uint32_t hb = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x, y}, bf16x2));
    if (nan)
      c[kBf16] += !bf16_is_nan(hb & 0xffffu) + !bf16_is_nan(hb >> 16);
    else
      c[kBf16] += ((hb & 0xffffu) != f32_to_bf16_rne(x)) + ((hb >> 16) != f32_to_bf16_rne(y));
    ++c[kValues];
  }
  // fp8 decode: all 256 codes through both halves of v_cvt_pk_f32_fp8
  if (first < 256) {
    const uint32_t code = (uint32_t)first;
    const int word = (int)(code | (code << 8) | (code << 16) | (code << 24));
    const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(word, false);
    const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(word, true);
    const float want = e4m3fn_to_f32(code);
    const float got[4] = {lo.x, lo.y, hi.x, hi.y};
    for (int k = 0; k < 4; ++k)
      c[kDecode] += (want != want) ? (got[k] == got[k]) : (f32_bits(got[k]) != f32_bits(want));
    // and straight to bf16 through v_cvt_scalef32_pk_bf16_fp8 at scale 1 (the
    // decode attention's K operand): every e4m3fn value is a bf16 value, so
    // the result must be exact; the four bytes of the word hold four codes
    const uint32_t codes[4] = {code, code ^ 0x55u, code ^ 0xaau, code ^ 0xffu};
    const int mixed = (int)(codes[0] | (codes[1] << 8) | (codes[2] << 16) | (codes[3] << 24));
    const uint32_t b_lo = __builtin_bit_cast(
        uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(mixed, 1.0f, false));
    const uint32_t b_hi = __builtin_bit_cast(
        uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(mixed, 1.0f, true));
    const uint32_t bgot[4] = {b_lo & 0xffffu, b_lo >> 16, b_hi & 0xffffu, b_hi >> 16};
    for (int k = 0; k < 4; ++k) {
      const float w = e4m3fn_to_f32(codes[k]);
      c[kDecode] += (w != w) ? !bf16_is_nan(bgot[k]) : (bgot[k] != f32_to_bf16_rne(w));
    }
  }
  // division: absmax bf16 pattern in the high 16 bits of v (all non-negative
  // patterns: finite, +inf and the NaNs), x in the low 16
  for (unsigned long long v = first; v < (0x8000ull << 16); v += stride) {
    const float amax_raw = bits_f32((uint32_t)(v >> 16) << 16);
    const float x = bits_f32((uint32_t)(v & 0xffffu) << 16);
    const bool nan_row = amax_raw != amax_raw;  // a NaN absmax: x may be anything
    if (!nan_row && (x != x)) continue;
    const float ax = x < 0.0f ? -x : x;
    if (!nan_row && ax > amax_raw) continue;
    const float amax = amax_raw < 1e-12f ? 1e-12f : amax_raw;
    const float b = amax / 448.0f;
    const float want = x / b;
    const float got = div_by_recip(x, b, 1.0f / b);
    const float aw = want < 0.0f ? -want : want;
    c[kDivQuot] += aw >= 0.000244140625f && f32_bits(want) != f32_bits(got);
    c[kDivCode] += !same_fp8(f32_to_e4m3fn(clamp448(want)), f32_to_e4m3fn(clamp448(got)));
    ++c[kPairs];
  }
  for (int k = 0; k < kCounters; ++k)
    if (c[k]) atomicAdd(&acc[k], c[k]);
  __syncthreads();
  if (threadIdx.x < kCounters && acc[threadIdx.x]) atomicAdd(&out[threadIdx.x], acc[threadIdx.x]);
}

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int mkv_check_conversions(uint64_t* counts, void* stream) {
  clear_error();
  MKV_REQUIRE(counts, MKV_E_INVALID, "mkv_check_conversions: null pointer");
  hipLaunchKernelGGL(check_conversions_kernel, dim3(4096), dim3(256), 0, as_stream(stream),
                     (unsigned long long*)counts);
  return check_launch("mkv_check_conversions");
}
