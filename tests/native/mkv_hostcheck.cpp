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
