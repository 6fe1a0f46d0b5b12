// Sampler tail: top-p filter, temperature and Gumbel-max draw over one row's
// descending candidates, executed by one wave64.
#pragma once
#include <float.h>
#include <math.h>

#include "tx_common.h"
#include "tx_math.h"

namespace tx {

// Gumbel noise of candidate token `id` in row `row_ctr`: threefry2x32 on the
// counter (0, row * vocab + id) (sparse_random.py:49-57,75-84).
__device__ __forceinline__ float candidate_noise(uint32_t k0, uint32_t k1, uint32_t row_ctr, uint32_t vocab,
                                                 int32_t id) {
  uint32_t o0, o1;
  threefry2x32(k0, k1, 0u, row_ctr * vocab + (uint32_t)id, o0, o1);
  return gumbel_from_bits(o0 ^ o1);
}

// Softmax numerator exp(v - v0) of a candidate (top_p_mask, sampling.py:45).
__device__ __forceinline__ float candidate_exp(float v, float v0) {
#pragma clang fp contract(off)
  return tx_expf(v - v0);
}

// ---------------------------------------------------------------------------
// Sampler tail on one row's sorted candidates, executed by one wave, in two
// parts so that the Gumbel noise can be computed by other waves meanwhile.
// Position p = h*64 + lane < K (K <= 128) holds value v[h], token id[h],
// numerator e[h] = exp(v - v[0]) and noise g[h].  Restates
// top_p_and_sample_arrays (sampling.py:65-115), top_p_mask (sampling.py:25-62),
// the (8,128)-tile cumsum order (cumsum.py:21-53) and max_arrays' tie rule
// (bitonic_top_k.py:43-97).
// ---------------------------------------------------------------------------

// Top-p threshold: probs = e / sum(e) (sum as a stride-halving tree over 128
// zero-padded slots), inclusive cumsum (Hillis-Steele inside 8-slot tiles,
// then the running total of earlier tiles added sequentially),
// t = #(cumsum < p), threshold v[t], or 0 when t == K (the out-of-range
// gather of take_along_axis_arrays).
__device__ __forceinline__ float top_p_threshold(const float v[2], const float e_in[2], int K, float top_p) {
#pragma clang fp contract(off)
  const int l = lane_id();
  const bool in[2] = {l < K, l + kWave < K};
  float e[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) e[h] = in[h] ? e_in[h] : 0.0f;
  float s = e[0] + e[1];
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) s = s + lane_xor_f(s, d);
  float c[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) c[h] = e[h] / s;
#pragma unroll
  for (int sh = 1; sh < 8; sh <<= 1) {
    const bool ok = (l & 7) >= sh;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float u = row_shr_f(c[h], sh);
      c[h] = c[h] + (ok ? u : 0.0f);
    }
  }
  // Tile g's total is its last slot (register g / 8, lane 8 (g % 8) + 7).  The
  // totals are read out first (independent readlanes), then summed in order
  // (carry_g = t_0 + ... + t_{g-1}, one add after the other), and each lane
  // picks the carries of its two tiles.
  const int tile0 = l >> 3;  // tile of register 0; register 1 is tile0 + 8
  float tt[16];
#pragma unroll
  for (int g = 0; g < 16; ++g) tt[g] = readlane_f(g < 8 ? c[0] : c[1], (g & 7) * 8 + 7);
  float carry[16];
  carry[0] = 0.0f;
  float run = tt[0];
#pragma unroll
  for (int g = 1; g < 16; ++g) {
    carry[g] = run;
    run = run + tt[g];
  }
  float carry0 = carry[0], carry1 = carry[8];
#pragma unroll
  for (int g = 1; g < 8; ++g) {
    carry0 = tile0 == g ? carry[g] : carry0;
    carry1 = tile0 == g ? carry[g + 8] : carry1;
  }
  if (tile0 != 0) c[0] = c[0] + carry0;
  c[1] = c[1] + carry1;
  const int t = __popcll(__ballot(in[0] && c[0] < top_p)) + __popcll(__ballot(in[1] && c[1] < top_p));
  const float vt = readlane_f(t < kWave ? v[0] : v[1], t & (kWave - 1));
  return t < K ? vt : 0.0f;
}

// Keep v >= thr (others become mask_val), divide by the temperature, add the
// noise and return the token of the maximum score; ties go to the largest
// bit-reversed position over log2(P) bits, P = max(8, pow2ceil(K)), with
// finfo.min / INT32_MIN padding as max_arrays pads.  T < 1e-5: greedy id[0].
__device__ __forceinline__ int32_t gumbel_argmax(const float v[2], const int32_t id[2], const float g[2], int K,
                                                 float thr, float temp, float mask_val) {
#pragma clang fp contract(off)
  const int l = lane_id();
  int P = 8;
  while (P < K) P <<= 1;
  int pbits = 0;
  while ((1 << pbits) < P) ++pbits;
  // One u64 key per slot: the score as an order-preserving integer (-0 as +0)
  // above the bit-reversed position, so the largest key is the largest score
  // with ties to the largest bit-reversed position; slots past P (which
  // max_arrays never sees) get key 0 and never win.
  uint64_t best = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int p = h * kWave + l;
    float sc = -FLT_MAX;  // padding slot of max_arrays (K <= p < P)
    if (p < K) {
      const float masked = v[h] >= thr ? v[h] : mask_val;
      const float scaled = masked / temp;
      sc = scaled + g[h];
    }
    uint32_t sb = __float_as_uint(sc);
    sb = sb == 0x80000000u ? 0u : sb;
    const uint32_t ord = sb ^ ((uint32_t)((int32_t)sb >> 31) | 0x80000000u);
    const uint64_t key = p < P ? (((uint64_t)ord << 32) | bitrev((uint32_t)p, pbits)) : 0ull;
    best = key > best ? key : best;
  }
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) {
    const uint64_t o = shfl_xor_u64(best, d);
    best = o > best ? o : best;
  }
  const int pw = (int)bitrev((uint32_t)best, pbits);  // the winning slot (uniform)
  const int32_t wid = (int32_t)readlane_u32((uint32_t)(pw < kWave ? id[0] : id[1]), pw & (kWave - 1));
  const int32_t best_i = pw < K ? wid : INT32_MIN;
  const int32_t greedy = (int32_t)readlane_u32((uint32_t)id[0], 0);
  return temp < 1e-5f ? greedy : best_i;
}

}  // namespace tx
