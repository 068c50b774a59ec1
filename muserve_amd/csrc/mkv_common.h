// mkv_common.h — helpers shared by the gfx950 kernels and by host-side checks.
//
// Everything here is plain integer/float arithmetic that compiles both as HIP
// device code (hipcc) and as ordinary C++ (g++), so the exact same encoders
// that run on the GPU can be compared exhaustively against the reference
// semantics on the CPU.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define MKV_HD __host__ __device__ __forceinline__
#else
#define MKV_HD static inline
#endif

namespace mkv {

MKV_HD uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
MKV_HD float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

// ---------------------------------------------------------------------------
// fp32 -> OCP fp8 e4m3fn, round to nearest even, non-saturating.
//
// e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa bits; no infinities; the
// only NaN codes are S.1111.111; largest finite 448 = 1.75*2^8; smallest
// normal 2^-6; subnormals m*2^-9, m=1..7. Like torch's .to(float8_e4m3fn),
// magnitudes that round above 448 become NaN (0x7F|sign): saturation is the
// caller's clamp (muserve/model/qwen35_layer_v2.py:84). NaN in -> 0x7F|sign.
// ---------------------------------------------------------------------------
MKV_HD uint8_t f32_to_e4m3fn(float x) {
  const uint32_t u = f32_bits(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a >= 0x43f00000u) return (uint8_t)(sign | 0x7fu);  // >= 480, inf, NaN
  const int e = (int)(a >> 23) - 127;                      // unbiased exponent
  if (e >= -6) {
    // fp8 normal: keep the top 3 of 23 mantissa bits, RNE on the other 20.
    uint32_t q = ((uint32_t)(e + 7) << 3) | ((a >> 20) & 7u);
    const uint32_t rem = a & 0xfffffu;
    q += (rem > 0x80000u) | ((rem == 0x80000u) & (q & 1u));  // carry may bump the exponent
    return (uint8_t)(sign | q);  // q == 0x7f here only for |x| in (464,480): NaN, as torch
  }
  if (e < -10) return (uint8_t)sign;  // |x| < 2^-10: rounds to (signed) zero
  // fp8 subnormal: m = RNE(|x| * 2^9) in [0, 8]; m == 8 encodes 2^-6 (0x08).
  const uint32_t sig = (a & 0x7fffffu) | 0x800000u;  // 24-bit significand
  const int shift = 14 - e;                           // 21..24
  uint32_t m = sig >> shift;
  const uint32_t rem = sig & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  m += (rem > half) | ((rem == half) & (m & 1u));
  return (uint8_t)(sign | m);
}

// OCP fp8 e4m3fn -> fp32 (exact).
MKV_HD float e4m3fn_to_f32(uint32_t q) {
  const uint32_t sign = (q & 0x80u) << 24;
  const uint32_t e = (q >> 3) & 0xfu;
  const uint32_t m = q & 7u;
  if (e == 0xfu && m == 7u) return bits_f32(sign | 0x7fc00000u);
  if (e == 0) {  // m * 2^-9
    return bits_f32(sign | f32_bits((float)m * 0.001953125f));
  }
  return bits_f32(sign | ((e + 120u) << 23) | (m << 20));
}

// x / b, correctly rounded, given y = 1/b correctly rounded (Markstein's
// correction step: q = RN(x*y) is within an ulp of x/b, r = x - q*b is exact
// through the fma, and RN(q + r*y) = RN(x/b)). Intermediates must be normal,
// which holds wherever the quotient can reach an fp8 code other than +-0. The
// step is skipped when r is 0 (q is exact; this also keeps the sign of -0) or
// NaN, which happens only for b = inf (y = 0: q = x*0 is already x/b, +-0 or
// NaN for x = +-inf) or b = NaN (q is NaN), so no separate path is needed.
// The fp8 quantiser's whole domain (every bf16 row absmax, including inf and
// NaN, as divisor source; every bf16 x with |x| <= absmax) is checked
// exhaustively against x / b, on the CPU and on the device.
MKV_HD float div_by_recip(float x, float b, float y) {
#pragma clang fp contract(off)
  const float q = x * y;
  const float r = __builtin_fmaf(-q, b, x);
  const float ar = r < 0.0f ? -r : r;
  return ar > 0.0f ? __builtin_fmaf(r, y, q) : q;
}

// e4m3fn codes equal, counting every NaN code (0x7F, 0xFF) as equal.
MKV_HD bool same_fp8(uint32_t a, uint32_t b) {
  return a == b || ((a & 0x7fu) == 0x7fu && (b & 0x7fu) == 0x7fu);
}

// fp32 -> bf16 bits, round to nearest even; every NaN becomes 0x7FC0 (the
// conversion torch's .to(torch.bfloat16) performs).
MKV_HD uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// ---------------------------------------------------------------------------
// SHA-256 compression function, FIPS 180-4 section 6.2.2.
// ---------------------------------------------------------------------------
MKV_HD uint32_t rotr32(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

// x ^ y ^ z. On gfx950 one v_bitop3_b32 (truth table 0x96); the compiler
// otherwise emits two XORs for each of the 4 sigma functions of every round.
MKV_HD uint32_t xor3(uint32_t x, uint32_t y, uint32_t z) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_bitop3_b32(x, y, z, 0x96);
#else
  return x ^ y ^ z;
#endif
}

MKV_HD uint32_t bswap32(uint32_t x) {
  return (x >> 24) | ((x >> 8) & 0xff00u) | ((x << 8) & 0xff0000u) | (x << 24);
}

constexpr uint32_t kSha256K[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u,
    0x923f82a4u, 0xab1c5ed5u, 0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u,
    0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u, 0xe49b69c1u, 0xefbe4786u,
    0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u,
    0x06ca6351u, 0x14292967u, 0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u,
    0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u, 0xa2bfe8a1u, 0xa81a664bu,
    0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au,
    0x5b9cca4fu, 0x682e6ff3u, 0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u,
    0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

struct Sha256 {
  uint32_t h[8];
};

MKV_HD void sha256_init(Sha256& s) {
  s.h[0] = 0x6a09e667u; s.h[1] = 0xbb67ae85u; s.h[2] = 0x3c6ef372u; s.h[3] = 0xa54ff53au;
  s.h[4] = 0x510e527fu; s.h[5] = 0x9b05688cu; s.h[6] = 0x1f83d9abu; s.h[7] = 0x5be0cd19u;
}

// One 64-byte block given as 16 big-endian message words.
MKV_HD void sha256_compress(Sha256& s, const uint32_t blk[16]) {
  uint32_t w[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) w[i] = blk[i];
  uint32_t a = s.h[0], b = s.h[1], c = s.h[2], d = s.h[3];
  uint32_t e = s.h[4], f = s.h[5], g = s.h[6], h = s.h[7];
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    uint32_t wi;
    if (i < 16) {
      wi = w[i];
    } else {
      const uint32_t w15 = w[(i - 15) & 15], w2 = w[(i - 2) & 15];
      const uint32_t s0 = xor3(rotr32(w15, 7), rotr32(w15, 18), w15 >> 3);
      const uint32_t s1 = xor3(rotr32(w2, 17), rotr32(w2, 19), w2 >> 10);
      wi = w[i & 15] = w[i & 15] + s0 + w[(i - 7) & 15] + s1;
    }
    const uint32_t S1 = xor3(rotr32(e, 6), rotr32(e, 11), rotr32(e, 25));
    const uint32_t ch = (e & f) ^ (~e & g);
    const uint32_t t1 = h + S1 + ch + kSha256K[i] + wi;
    const uint32_t S0 = xor3(rotr32(a, 2), rotr32(a, 13), rotr32(a, 22));
    const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
    const uint32_t t2 = S0 + maj;
    h = g; g = f; f = e; e = d + t1;
    d = c; c = b; b = a; a = t1 + t2;
  }
  s.h[0] += a; s.h[1] += b; s.h[2] += c; s.h[3] += d;
  s.h[4] += e; s.h[5] += f; s.h[6] += g; s.h[7] += h;
}

// The padding block of a message of message_bytes bytes whose length is a
// whole number of 64-byte blocks: 0x80, zeros, the 64-bit big-endian bit count.
MKV_HD void sha256_pad_block(uint32_t pad[16], uint64_t message_bytes) {
#pragma unroll
  for (int i = 0; i < 16; ++i) pad[i] = 0;
  pad[0] = 0x80000000u;
  const uint64_t bits = message_bytes * 8u;
  pad[14] = (uint32_t)(bits >> 32);
  pad[15] = (uint32_t)bits;
}

// Digest prefix of a message whose length is a whole number of 64-byte blocks
// already absorbed into `s`: the padding is one full block (0x80, zeros, the
// 64-bit big-endian bit length). Returns the first 8 digest bytes as a
// big-endian u64, i.e. int(hexdigest()[:16], 16).
MKV_HD uint64_t sha256_final_aligned_u64(const Sha256& s, uint64_t message_bytes) {
  uint32_t pad[16];
  sha256_pad_block(pad, message_bytes);
  Sha256 t = s;
  sha256_compress(t, pad);
  return ((uint64_t)t.h[0] << 32) | t.h[1];
}

}  // namespace mkv
