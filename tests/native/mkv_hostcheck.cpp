// Host (g++) build of the encoders in muserve_amd/csrc/mkv_common.h, so the
// exact code the kernels run can be compared exhaustively with torch on a CPU.
// Test infrastructure: loaded only by tests/.
#include <stdint.h>

#include "mkv_common.h"

extern "C" {

// e4m3fn codes of every float32 whose bit pattern is in [lo, hi).
void hc_e4m3fn_encode_bits(uint64_t lo, uint64_t hi, uint8_t* out) {
  for (uint64_t u = lo; u < hi; ++u) out[u - lo] = mkv::f32_to_e4m3fn(mkv::bits_f32((uint32_t)u));
}

void hc_e4m3fn_encode(const float* x, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = mkv::f32_to_e4m3fn(x[i]);
}

void hc_e4m3fn_decode(const uint8_t* q, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = mkv::e4m3fn_to_f32(q[i]);
}

void hc_bf16_rne(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = mkv::f32_to_bf16_rne(x[i]);
}

// Per-page prefix hashes of one request, like mkv_block_hash_sha256.
void hc_page_hashes(const uint8_t* tokens, int64_t ntok, int32_t token_bytes, uint64_t* out) {
  mkv::Sha256 s;
  mkv::sha256_init(s);
  const int64_t pages = ntok / 16;
  const int words = token_bytes * 16 / 4;
  for (int64_t i = 0; i < pages; ++i) {
    for (int blk = 0; blk < words / 16; ++blk) {
      uint32_t w[16];
      for (int j = 0; j < 16; ++j) {
        const uint8_t* p = tokens + (i * words + blk * 16 + j) * 4;
        w[j] = ((uint32_t)p[0] << 24) | ((uint32_t)p[1] << 16) | ((uint32_t)p[2] << 8) | p[3];
      }
      mkv::sha256_compress(s, w);
    }
    out[i] = mkv::sha256_final_aligned_u64(s, (uint64_t)(i + 1) * 16 * token_bytes);
  }
}

}  // extern "C"

// Exhaustive check of the fp8 quantiser's division over its reachable domain:
// for every non-negative bf16 absmax a (the divisor is
// b = max(a, 1e-12f) / 448) and every bf16 x with |x| <= a, compares
// div_by_recip(x, b, 1/b) with x / b: the e4m3fn code of the clamped quotient
// everywhere, and the quotient bits wherever |x / b| >= 2^-12 (below that the
// residual may underflow, and every such quotient encodes to +-0). Returns the
// number of code mismatches; quotient mismatches go to *quot_bad.
// Infinite and NaN absmax rows are included (codes compared with every NaN
// code equal to every other).
extern "C" int64_t hc_check_div_by_recip(uint32_t a_lo, uint32_t a_hi, int64_t* quot_bad,
                                         int64_t* pairs) {
  int64_t bad = 0, qb = 0, n = 0;
  for (uint32_t ah = a_lo; ah < a_hi; ++ah) {  // bf16 bit patterns of the absmax
    const float a = mkv::bits_f32(ah << 16);
    const bool nan_row = !(a == a);  // a NaN absmax: the row's x may be anything
    const float amax = a < 1e-12f ? 1e-12f : a;
    const float b = amax / 448.0f;
    const float y = 1.0f / b;
    for (uint32_t xh = 0; xh < 65536; ++xh) {
      const float x = mkv::bits_f32(xh << 16);
      if (!nan_row && !(x == x)) continue;
      const float ax = x < 0 ? -x : x;
      if (!nan_row && ax > a) continue;
      const float want = x / b;
      const float got = mkv::div_by_recip(x, b, y);
      ++n;
      const float aw = want < 0 ? -want : want;
      if (aw >= 0.000244140625f && mkv::f32_bits(want) != mkv::f32_bits(got)) ++qb;
      auto cl = [](float v) { return v < -448.0f ? -448.0f : (v > 448.0f ? 448.0f : v); };
      if (!mkv::same_fp8(mkv::f32_to_e4m3fn(cl(want)), mkv::f32_to_e4m3fn(cl(got)))) ++bad;
    }
  }
  *quot_bad = qb;
  *pairs = n;
  return bad;
}

