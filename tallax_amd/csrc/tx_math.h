// Single-precision exp / log and the Threefry-2x32 counter hash used by the
// sampler, written from the mathematics so that a plain numpy float32
// restatement reproduces every result bit for bit:
//   * every operation is one IEEE-754 binary32 op (add, sub, mul, correctly
//     rounded divide, round-to-nearest-even rint) -- no fused multiply-add.
//     The whole library is compiled with -ffp-contract=off and the pragmas
//     below repeat that locally;
//   * the constants are the float32 roundings of ln 2, log2 e, 1/n! and 2/(2n+1).
//
// exp: Cody & Waite (1980) range reduction x = n ln2 + r, |r| <= ln2/2, with
// ln2 split in a 12-trailing-zero-bit head (n*head is exact for |n| < 2^12) and
// a tail; exp(r) = 1 + (r + r^2 q(r)) with q the degree-5 Taylor tail in
// Horner form (so the only rounding of size ~ulp(1) is the final add); 2^n applied
// as one or two exact power-of-two scalings (two for results near the
// subnormal range so that the only rounding is the final one).
//
// log: x = 2^e m with m in [sqrt(1/2), sqrt(2)), f = m - 1 (exact by Sterbenz),
// s = f/(2+f), log(1+f) = 2 atanh(s) = f - (f^2/2 - s (f^2/2 + R(s^2))) with
// R(z) = z (2/3 + z (2/5 + z (2/7 + z (2/9 + z (2/11 + z 2/13))))).
//
// Threefry-2x32 with 20 rounds: Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC'11 (rotation constants and key schedule as
// published there); pinned by the Random123 / JAX known-answer vectors in the
// test suite.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tx {

#define TX_F(h) __uint_as_float(h##u)

__device__ __forceinline__ float tx_expf(float x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  const float xc = fminf(fmaxf(x, -120.0f), 100.0f);
  const float n = rintf(xc * TX_F(0x3fb8aa3b));            // log2(e)
  const float r = (xc - n * TX_F(0x3f317000)) - n * TX_F(0x3805fdf4);  // ln2 head, tail
  // exp(r) = 1 + (r + r^2 q(r)), q(r) = 1/2 + r/3! + ... + r^5/7!
  float q = TX_F(0x39500d01);                               // 1/7!
  q = q * r + TX_F(0x3ab60b61);                             // 1/6!
  q = q * r + TX_F(0x3c088889);                             // 1/5!
  q = q * r + TX_F(0x3d2aaaab);                             // 1/4!
  q = q * r + TX_F(0x3e2aaaab);                             // 1/3!
  q = q * r + 0.5f;
  const float p = 1.0f + ((r * r) * q + r);
  const int ni = (int)n;
  if (ni >= -126 && ni <= 127) return p * __int_as_float((ni + 127) << 23);
  const int n1 = ni / 2;
  const int n2 = ni - n1;
  return (p * __int_as_float((n1 + 127) << 23)) * __int_as_float((n2 + 127) << 23);
}

__device__ __forceinline__ float tx_logf(float x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  if (x < 0.0f) return __uint_as_float(0x7fc00000u);
  if (x == 0.0f) return __uint_as_float(0xff800000u);
  uint32_t b = __float_as_uint(x);
  if (b == 0x7f800000u) return x;
  int e = 0;
  if (b < 0x00800000u) {  // subnormal: scale by 2^23 (exact)
    x = x * 8388608.0f;
    b = __float_as_uint(x);
    e = -23;
  }
  e += (int)(b >> 23) - 127;
  float m = __uint_as_float((b & 0x007fffffu) | 0x3f800000u);
  if (m > TX_F(0x3fb504f3)) {  // sqrt(2)
    m = m * 0.5f;
    e += 1;
  }
  const float f = m - 1.0f;
  const float s = f / (2.0f + f);
  const float z = s * s;
  float R = TX_F(0x3e1d89d9);             // 2/13
  R = R * z + TX_F(0x3e3a2e8c);           // 2/11
  R = R * z + TX_F(0x3e638e39);           // 2/9
  R = R * z + TX_F(0x3e924925);           // 2/7
  R = R * z + TX_F(0x3ecccccd);           // 2/5
  R = R * z + TX_F(0x3f2aaaab);           // 2/3
  R = R * z;
  const float hfsq = (0.5f * f) * f;
  const float dk = (float)e;
  return dk * TX_F(0x3f317000) - ((hfsq - (s * (hfsq + R) + dk * TX_F(0x3805fdf4))) - f);
}

__device__ __forceinline__ uint32_t rotl32(uint32_t v, int r) { return (v << r) | (v >> (32 - r)); }

// Threefry-2x32-20 of counter (c0, c1) under key (k0, k1).
__device__ __forceinline__ void threefry2x32(uint32_t k0, uint32_t k1, uint32_t c0, uint32_t c1,
                                             uint32_t& o0, uint32_t& o1) {
  const uint32_t ks[3] = {k0, k1, k0 ^ k1 ^ 0x1BD11BDAu};
  constexpr int R[8] = {13, 15, 26, 6, 17, 29, 16, 24};
  uint32_t x0 = c0 + ks[0];
  uint32_t x1 = c1 + ks[1];
#pragma unroll
  for (int blk = 0; blk < 5; ++blk) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x0 += x1;
      x1 = rotl32(x1, R[(blk & 1) * 4 + i]);
      x1 ^= x0;
    }
    x0 += ks[(blk + 1) % 3];
    x1 += ks[(blk + 2) % 3] + (uint32_t)(blk + 1);
  }
  o0 = x0;
  o1 = x1;
}

// float32 in [0, 1) from 32 random bits: the 23 high bits become the mantissa
// of a number in [1, 2), then 1 is subtracted (tallax/_src/sparse_random.py:7-41).
__device__ __forceinline__ float bits_to_unit(uint32_t bits) {
#pragma clang fp contract(off)
  return __uint_as_float((bits >> 9) | 0x3f800000u) - 1.0f;
}

// Gumbel noise -log(-log(u)) for u = max(tiny, unit*(1 - tiny) + tiny)
// (sparse_random.py:43-64 with minval = finfo(f32).tiny, maxval = 1, and :84).
__device__ __forceinline__ float gumbel_from_bits(uint32_t bits) {
#pragma clang fp contract(off)
  const float tiny = __uint_as_float(0x00800000u);
  const float scale = 1.0f - tiny;
  const float u = fmaxf(tiny, bits_to_unit(bits) * scale + tiny);
  return -tx_logf(-tx_logf(u));
}

#undef TX_F

}  // namespace tx
