// Wave64 bitonic networks held in registers.
//
// A "run" is 128 composites (u32 or u64) spread over one wave, two per lane: element
// i lives in lane i % 64, register i / 64.  Compare-exchange partners at
// distance 64 sit in the same lane; smaller distances are exchanged across
// lanes with DPP / v_permlane*_swap (lane_xor), so neither LDS nor barriers
// are involved.
#pragma once
#include "tx_common.h"

namespace tx {

// One compare-exchange: keep own value if (own > other) == keep_max.
__device__ __forceinline__ uint32_t cx_u32(uint32_t v, uint32_t o, bool keep_max) {
  return ((v > o) == keep_max) ? v : o;
}

// Sort 64 u32 values (one per lane) in descending order.
__device__ __forceinline__ uint32_t wave_sort64_u32_desc(uint32_t v) {
  const int l = lane_id();
#pragma unroll
  for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride >= 1; stride >>= 1) {
      const bool desc = (l & size) == 0;
      const bool lower = (l & stride) == 0;
      v = cx_u32(v, lane_xor(v, stride), lower == desc);
    }
  }
  return v;
}

__device__ __forceinline__ uint32_t lane_xor_c(uint32_t v, int d) { return lane_xor(v, d); }
__device__ __forceinline__ uint64_t lane_xor_c(uint64_t v, int d) { return shfl_xor_u64(v, d); }
__device__ __forceinline__ uint32_t lane_rev_c(uint32_t v) { return lane_rev(v); }
__device__ __forceinline__ uint64_t lane_rev_c(uint64_t v) {
  return ((uint64_t)lane_rev((uint32_t)(v >> 32)) << 32) | lane_rev((uint32_t)v);
}
template <typename C>
__device__ __forceinline__ C cx(C v, C o, bool keep_max) {
  return ((v > o) == keep_max) ? v : o;
}

// Sort 64 composites (one per lane) in descending order.
template <typename C>
__device__ __forceinline__ C wave_sort64_desc(C v) {
  const int l = lane_id();
#pragma unroll
  for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride >= 1; stride >>= 1) {
      const bool desc = (l & size) == 0;
      const bool lower = (l & stride) == 0;
      v = cx(v, lane_xor_c(v, stride), lower == desc);
    }
  }
  return v;
}

// Sort a run of 128 composites (u32 or u64) in descending order.
template <typename C>
__device__ __forceinline__ void wave_sort128_desc(C c[2]) {
  const int l = lane_id();
#pragma unroll
  for (int size = 2; size <= 2 * kWave; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride >= 1; stride >>= 1) {
      if (stride == kWave) {  // only at size 128, which is sorted descending
        const bool gt = c[0] > c[1];
        const C hi = gt ? c[0] : c[1];
        const C lo = gt ? c[1] : c[0];
        c[0] = hi;
        c[1] = lo;
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int i = h * kWave + l;
          const bool desc = (i & size) == 0;
          const bool lower = (i & stride) == 0;
          c[h] = cx(c[h], lane_xor_c(c[h], stride), lower == desc);
        }
      }
    }
  }
}

// Bitonic merge of a bitonic run into descending order.
template <typename C>
__device__ __forceinline__ void wave_bitonic_merge128_desc(C c[2]) {
  const int l = lane_id();
  const bool gt = c[0] > c[1];
  const C hi = gt ? c[0] : c[1];
  const C lo = gt ? c[1] : c[0];
  c[0] = hi;
  c[1] = lo;
#pragma unroll
  for (int stride = kWave / 2; stride >= 1; stride >>= 1) {
    const bool lower = (l & stride) == 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) c[h] = cx(c[h], lane_xor_c(c[h], stride), lower);
  }
}

// a <- the 128 largest of a u b (both descending runs), descending.
// Merge-and-discard: max(a[i], b[127 - i]) is bitonic and holds the top 128.
template <typename C>
__device__ __forceinline__ void wave_merge128_desc(C a[2], const C b[2]) {
  const C rb0 = lane_rev_c(b[1]);  // b[127 - lane]
  const C rb1 = lane_rev_c(b[0]);  // b[63 - lane]
  a[0] = a[0] > rb0 ? a[0] : rb0;
  a[1] = a[1] > rb1 ? a[1] : rb1;
  wave_bitonic_merge128_desc(a);
}

// The 64 largest of a u b (descending runs of 64, one entry per lane),
// descending: max(a[i], b[63 - i]) is bitonic and holds them.
template <typename C>
__device__ __forceinline__ C wave_merge64_desc(C a, C b) {
  const int l = lane_id();
  const C rb = lane_rev_c(b);
  C v = a > rb ? a : rb;
#pragma unroll
  for (int stride = kWave / 2; stride >= 1; stride >>= 1) v = cx(v, lane_xor_c(v, stride), (l & stride) == 0);
  return v;
}

}  // namespace tx
