// Wave64 bitonic networks held in registers.
//
// A "run" is 128 u64 composites spread over one wave, two per lane: element
// i lives in lane i % 64, register i / 64.  Compare-exchange partners at
// distance 64 sit in the same lane; smaller distances are exchanged across
// lanes with ds_bpermute (HIP __shfl_xor), so no LDS storage and no barriers
// are involved.
#pragma once
#include "tx_common.h"

namespace tx {

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t umin64(uint64_t a, uint64_t b) { return a > b ? b : a; }

// Sort 64 u32 values (one per lane) in descending order.
__device__ __forceinline__ uint32_t wave_sort64_u32_desc(uint32_t v) {
  const int l = lane_id();
#pragma unroll
  for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride >= 1; stride >>= 1) {
      const uint32_t o = (uint32_t)__shfl_xor((int)v, stride, kWave);
      const bool desc = (l & size) == 0;
      const bool lower = (l & stride) == 0;
      const bool keep_max = lower == desc;
      v = keep_max ? (v > o ? v : o) : (v > o ? o : v);
    }
  }
  return v;
}

// Sort a run of 128 composites in descending order.
__device__ __forceinline__ void wave_sort128_desc(uint64_t c[2]) {
  const int l = lane_id();
#pragma unroll
  for (int size = 2; size <= 2 * kWave; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride >= 1; stride >>= 1) {
      if (stride == kWave) {  // only at size 128, which is sorted descending
        const uint64_t hi = umax64(c[0], c[1]);
        const uint64_t lo = umin64(c[0], c[1]);
        c[0] = hi;
        c[1] = lo;
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int i = h * kWave + l;
          const uint64_t o = shfl_xor_u64(c[h], stride);
          const bool desc = (i & size) == 0;
          const bool lower = (i & stride) == 0;
          c[h] = (lower == desc) ? umax64(c[h], o) : umin64(c[h], o);
        }
      }
    }
  }
}

// Bitonic merge of a bitonic run into descending order.
__device__ __forceinline__ void wave_bitonic_merge128_desc(uint64_t c[2]) {
  const int l = lane_id();
  const uint64_t hi = umax64(c[0], c[1]);
  const uint64_t lo = umin64(c[0], c[1]);
  c[0] = hi;
  c[1] = lo;
#pragma unroll
  for (int stride = kWave / 2; stride >= 1; stride >>= 1) {
    const bool lower = (l & stride) == 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint64_t o = shfl_xor_u64(c[h], stride);
      c[h] = lower ? umax64(c[h], o) : umin64(c[h], o);
    }
  }
}

__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
  const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)v, src, kWave);
  const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(v >> 32), src, kWave);
  return ((uint64_t)hi << 32) | lo;
}

// a <- the 128 largest of a u b (both descending runs), descending.
// Merge-and-discard: max(a[i], b[127 - i]) is bitonic and holds the top 128.
__device__ __forceinline__ void wave_merge128_desc(uint64_t a[2], const uint64_t b[2]) {
  const int l = lane_id();
  const uint64_t rb0 = shfl_u64(b[1], kWave - 1 - l);  // b[127 - l]
  const uint64_t rb1 = shfl_u64(b[0], kWave - 1 - l);  // b[63 - l]
  a[0] = umax64(a[0], rb0);
  a[1] = umax64(a[1], rb1);
  wave_bitonic_merge128_desc(a);
}

}  // namespace tx
