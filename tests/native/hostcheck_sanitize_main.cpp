// The shared arithmetic of muserve_amd/csrc/mkv_common.h (through the
// host-check functions of mkv_hostcheck.cpp), built by g++ with
// AddressSanitizer and UndefinedBehaviorSanitizer (tests/test_sanitizers.py):
// the fp8 encoder over a stride of all fp32 bit patterns and its boundary
// values, the decoder on every code (and re-encoding each finite value to its
// own code), bf16 rounding, the page-hash chain and the quantiser's divide on
// a block of divisors. Test infrastructure only.
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "mkv_hostcheck.cpp"

int main() {
  int failures = 0;
  // encoder: every 4099th bit pattern, then +-[0, 2^20) around the 448/480 and
  // subnormal boundaries
  uint64_t checksum = 0;
  for (uint64_t u = 0; u < (1ull << 32); u += 4099) checksum += mkv::f32_to_e4m3fn(mkv::bits_f32((uint32_t)u));
  static uint8_t codes[1 << 20];
  const uint32_t bases[] = {0x43e00000u, 0x43f00000u, 0x3a800000u, 0x3b000000u, 0x00000000u,
                            0xc3e00000u, 0x7f800000u};
  for (uint32_t b : bases) {
    hc_e4m3fn_encode_bits(b, (uint64_t)b + (1u << 20), codes);
    for (uint32_t i = 0; i < (1u << 20); ++i) checksum += codes[i];
  }
  // decoder on all 256 codes; every non-NaN value re-encodes to its own code
  uint8_t all[256];
  float vals[256];
  for (int i = 0; i < 256; ++i) all[i] = (uint8_t)i;
  hc_e4m3fn_decode(all, vals, 256);
  uint8_t back[256];
  hc_e4m3fn_encode(vals, back, 256);
  for (int i = 0; i < 256; ++i)
    if ((i & 0x7f) != 0x7f && back[i] != i) {
      fprintf(stderr, "code %#x decodes to %g and re-encodes to %#x\n", i, vals[i], back[i]);
      ++failures;
    }
  // bf16 rounding of the decoded values is exact (every e4m3fn value is a bf16)
  uint16_t bf[256];
  hc_bf16_rne(vals, bf, 256);
  for (int i = 0; i < 256; ++i)
    if ((i & 0x7f) != 0x7f && mkv::bits_f32((uint32_t)bf[i] << 16) != vals[i]) ++failures;
  // page hashes of a 1000-token request at 8 and 4 bytes per token: the chain
  // over the first k pages does not depend on later tokens
  static uint8_t tok[1000 * 8];
  for (int i = 0; i < 1000 * 8; ++i) tok[i] = (uint8_t)(i * 131 + 7);
  uint64_t h8[62], h4[62], h8short[10];
  hc_page_hashes(tok, 1000, 8, h8);
  hc_page_hashes(tok, 1000, 4, h4);
  hc_page_hashes(tok, 160, 8, h8short);
  for (int i = 0; i < 10; ++i)
    if (h8short[i] != h8[i]) ++failures;
  checksum += h8[61] ^ h4[61];
  // the quantiser's divide on 64 absmax values around 1.0 and the largest ones
  int64_t quot_bad = 0, pairs = 0;
  int64_t bad = hc_check_div_by_recip(0x3f80u, 0x3fc0u, &quot_bad, &pairs);
  int64_t qb2 = 0, p2 = 0;
  bad += hc_check_div_by_recip(0x7f40u, 0x7f80u, &qb2, &p2);
  if (bad || quot_bad || qb2) {
    fprintf(stderr, "divide: %lld code and %lld quotient mismatches\n", (long long)bad,
            (long long)(quot_bad + qb2));
    ++failures;
  }
  printf("hostcheck sanitize driver: %d failures, checksum %llx, %lld divide pairs\n", failures,
         (unsigned long long)checksum, (long long)(pairs + p2));
  return failures ? 1 : 0;
}
