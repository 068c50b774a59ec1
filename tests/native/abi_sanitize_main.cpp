// Host-side driver of every libmuserve_kv entry point's argument checking,
// built with AddressSanitizer and UndefinedBehaviorSanitizer on the host code
// (tests/test_sanitizers.py). Every call below must be rejected (or be a
// size-0 no-op) before any HIP call, so it runs without a GPU. Test
// infrastructure only.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "mkv.h"

static int failures = 0;

static void expect_rejected(const char* name, int rc) {
  const char* msg = mkv_last_error();
  if (rc >= 0 || msg == nullptr || msg[0] == '\0') {
    fprintf(stderr, "%s: expected an argument error, got %d (\"%s\")\n", name, rc, msg ? msg : "");
    ++failures;
  }
}

static void expect_ok(const char* name, int rc) {
  if (rc != MKV_OK) {
    fprintf(stderr, "%s: expected MKV_OK, got %d (\"%s\")\n", name, rc, mkv_last_error());
    ++failures;
  }
}

int main() {
  void* N = nullptr;
  int32_t err = 0;
  int32_t* E = &err;
  // null pointers with non-zero sizes
  expect_rejected("append_bf16", mkv_append_bf16(N, N, 0, 16, N, N, 0, 512, nullptr, 1, 1, 512, E, N));
  expect_rejected("gather_bf16", mkv_gather_bf16(N, N, 0, 4, nullptr, 4, 4, nullptr, nullptr, 1, 16,
                                                 nullptr, N, N, 0, 1, 512, E, N));
  expect_rejected("decode_slots", mkv_decode_slots(nullptr, nullptr, 4, 4, nullptr, 1, 4, nullptr, E, N));
  expect_rejected("step_plan", mkv_step_plan(nullptr, 4, 4, 1, nullptr, 1, nullptr, 1, 4, nullptr,
                                             nullptr, 1, nullptr, 4, 4, nullptr, nullptr, nullptr, E, N));
  expect_rejected("append_fp8", mkv_append_fp8(N, N, nullptr, nullptr, 0, 0, 16, N, N, 0, 512,
                                               nullptr, 1, 1, 1, 256, E, N));
  expect_rejected("gather_dequant_fp8",
                  mkv_gather_dequant_fp8(N, N, nullptr, nullptr, 0, 0, 4, nullptr, 4, 4, nullptr,
                                         nullptr, 1, 16, nullptr, N, N, 0, 1, 1, 256, E, N));
  expect_rejected("copy_blocks", mkv_copy_blocks(N, 0, 1, 4, 8192, nullptr, nullptr, 1, E, N));
  expect_rejected("state_gather", mkv_state_gather(N, 16, N, N, 0, N, 4, nullptr, 1, E, N));
  expect_rejected("state_scatter", mkv_state_scatter(N, 16, N, N, 0, N, 4, nullptr, 1, E, N));
  expect_rejected("gdn_conv_decode", mkv_gdn_conv_decode(N, 4, 2048, 4, nullptr, 1, N, N, 4, N, E, N));
  expect_rejected("gdn_decode_gather", mkv_gdn_decode_gather(N, 16, N, N, 2048, 4, 4, nullptr, 1, N,
                                                             N, 4, N, E, N));
  expect_rejected("pack_blocks", mkv_pack_blocks(N, 0, 1, 8192, 4, nullptr, 1, N, E, N));
  expect_rejected("unpack_blocks", mkv_unpack_blocks(N, 0, 1, 8192, 4, nullptr, 1, N, E, N));
  expect_rejected("zero_blocks", mkv_zero_blocks(N, 0, 1, 8192, 4, nullptr, 1, E, N));
  expect_rejected("zero_blocks overlap", mkv_zero_blocks(N, 16, 2, 8192, 4, nullptr, 1, E, N));
  expect_ok("zero_blocks empty", mkv_zero_blocks(N, 0, 1, 8192, 4, nullptr, 0, E, N));
  expect_rejected("block_hash", mkv_block_hash_sha256(N, nullptr, nullptr, 1, 8, nullptr, E, N));
  expect_rejected("bm_init", mkv_bm_init(N, 16, nullptr, N));
  expect_rejected("bm_step", mkv_bm_step(N, 16, nullptr, 1, 1, nullptr, nullptr, nullptr, nullptr, 4,
                                         4, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0,
                                         E, N));
  expect_rejected("hash_probe", mkv_hash_probe(N, 16, nullptr, nullptr, 1, nullptr, nullptr, E, N));
  expect_rejected("attention_bf16",
                  mkv_decode_attention_bf16(N, N, N, 4, 0, 1, 4, 256, nullptr, 4, 4, nullptr, 1,
                                            64, 0.0625f, N, N, 0, E, N));
  expect_rejected("attention_fp8",
                  mkv_decode_attention_fp8(N, N, N, nullptr, nullptr, 4, 0, 1, 4, 256, nullptr, 4,
                                           4, nullptr, 1, 64, 0.0625f, N, N, 0, E, N));
  expect_rejected("attention_contig", mkv_decode_attention_contig(N, N, N, 0, 1, 4, 256, 0,
                                                                  nullptr, 1, 64, 0.0625f, N, N,
                                                                  0, E, N));
  expect_rejected("prefill_attention", mkv_prefill_attention_bf16(N, N, N, 4, 1, 4, 256, nullptr, 0, 0, nullptr, nullptr, nullptr, 1, 16, 16, 0.0625f, 1, 1, 0, N, N, 0, E, N));
  expect_rejected("prefill_attention split", mkv_prefill_attention_bf16(N, N, N, 4, 1, 4, 256, nullptr, 0, 0, nullptr, nullptr, nullptr, 1, 16, 16, 0.0625f, 1, 4, 33, N, N, 0, E, N));
  if (mkv_prefill_attention_workspace_bytes(100, 4, 1) != 0 || mkv_prefill_attention_workspace_bytes(100, 4, 3) <= 0) ++failures;
  expect_rejected("check_conversions", mkv_check_conversions(nullptr, N));
  // negative sizes
  expect_rejected("append_bf16 negative", mkv_append_bf16(N, N, 0, 16, N, N, 0, 512, nullptr, -1, 1,
                                                          512, E, N));
  expect_rejected("step_plan negative", mkv_step_plan(nullptr, 4, 4, 1, nullptr, -1, nullptr, 0, 4,
                                                      nullptr, nullptr, 0, nullptr, 4, 4, nullptr,
                                                      nullptr, nullptr, E, N));
  expect_rejected("copy_blocks negative", mkv_copy_blocks(N, 0, 1, 4, 8192, nullptr, nullptr, -3, E, N));
  // size-0 calls return at once without touching any pointer
  expect_ok("decode_slots empty", mkv_decode_slots(nullptr, nullptr, 4, 4, nullptr, 0, 4, nullptr, E, N));
  expect_ok("step_plan empty", mkv_step_plan(nullptr, 4, 4, 1, nullptr, 0, nullptr, 0, 4, nullptr,
                                             nullptr, 0, nullptr, 4, 4, nullptr, nullptr, nullptr, E, N));
  expect_ok("copy_blocks empty", mkv_copy_blocks(N, 0, 1, 4, 8192, nullptr, nullptr, 0, E, N));
  // host-side sizing: the block manager's layout over many pool sizes
  for (int32_t p = 1; p <= (1 << 22); p = p * 3 + 1) {
    int64_t lay[10];
    memset(lay, 0, sizeof(lay));
    if (mkv_bm_layout(p, lay) != MKV_OK || lay[9] != mkv_bm_state_bytes(p)) {
      fprintf(stderr, "bm_layout(%d): inconsistent total\n", p);
      ++failures;
      continue;
    }
    // lay: table capacity, ring capacity, then the offsets of counters,
    // table, page records, free stack, ring, last-occurrence slots and
    // release-run scratch, then the total
    for (int i = 2; i < 9; ++i)
      if (lay[i] % 16 != 0 || (i > 2 && lay[i] < lay[i - 1]) || lay[i] > lay[9]) {
        fprintf(stderr, "bm_layout(%d): offset %d = %lld out of order or unaligned\n", p, i,
                (long long)lay[i]);
        ++failures;
      }
  }
  expect_rejected("bm_layout negative", mkv_bm_layout(-5, nullptr));
  if (mkv_bm_state_bytes(0) > 0 || mkv_bm_state_bytes(-1) > 0) {
    fprintf(stderr, "bm_state_bytes accepted an empty pool\n");
    ++failures;
  }
  for (int32_t b = 1; b <= 4096; b *= 4)
    for (int32_t len = 1; len <= (1 << 18); len *= 8)
      if (mkv_decode_attention_workspace_bytes(b, 1, 4, len) <= 0) {
        fprintf(stderr, "attention workspace(%d, %d) not positive\n", b, len);
        ++failures;
      }
  if (mkv_version() != MKV_ABI_VERSION) ++failures;
  printf("abi sanitize driver: %d failures\n", failures);
  return failures ? 1 : 0;
}
