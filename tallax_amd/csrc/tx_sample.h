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
  const int tile0 = l >> 3;  // tile of register 0; register 1 is tile0 + 8
  float carry0 = 0.0f, carry1 = 0.0f;
  float run = readlane_f(c[0], 7);
#pragma unroll
  for (int g = 1; g < 16; ++g) {
    if (tile0 == g) carry0 = run;
    if (tile0 + 8 == g) carry1 = run;
    const float tsg = readlane_f(g < 8 ? c[0] : c[1], (g & 7) * 8 + 7);
    run = run + tsg;
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
  float best_s = 0.0f;
  uint32_t best_b = 0;
  int32_t best_i = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int p = h * kWave + l;
    float sc;
    int32_t tok = id[h];
    if (p < K) {
      const float masked = v[h] >= thr ? v[h] : mask_val;
      const float scaled = masked / temp;
      sc = scaled + g[h];
    } else if (p < P) {
      sc = -FLT_MAX;
      tok = INT32_MIN;
    } else {
      sc = -INFINITY;
    }
    const uint32_t br = p < P ? bitrev((uint32_t)p, pbits) : 0u;
    if (h == 0 || sc > best_s || (sc == best_s && br > best_b)) {
      best_s = sc;
      best_b = br;
      best_i = tok;
    }
  }
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) {
    const float os = lane_xor_f(best_s, d);
    const uint32_t ob = lane_xor(best_b, d);
    const int32_t oi = (int32_t)lane_xor((uint32_t)best_i, d);
    if (os > best_s || (os == best_s && ob > best_b)) {
      best_s = os;
      best_b = ob;
      best_i = oi;
    }
  }
  const int32_t greedy = (int32_t)readlane_u32((uint32_t)id[0], 0);
  return temp < 1e-5f ? greedy : best_i;
}

}  // namespace tx
