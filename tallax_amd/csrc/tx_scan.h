// Scan helpers shared by cumsum and the fused softmax / top-k / cumsum
// kernel: the reference's per-tile Hillis-Steele order (cumsum.py:21-30) on
// 128-position tiles held two per lane (position p = h * 64 + lane).
#pragma once
#include "tx_common.h"

namespace tx {

template <typename T>
__device__ __forceinline__ T shfl_up_or_zero(T v, int s, int l) {
  // value of lane l - s (0 when l < s), via the LDS crossbar (no LDS memory)
  const int src = l - s;
  const int x = __builtin_amdgcn_ds_bpermute((src < 0 ? l : src) << 2, __builtin_bit_cast(int, v));
  return src < 0 ? (T)0 : __builtin_bit_cast(T, x);
}

// Inclusive prefix sum of an integer over the wave's 64 lanes: DPP row
// shifts (1, 2, 4, 8) inside each 16-lane row, then the totals of the rows
// below added through readlane -- VALU lane exchanges, no LDS crossbar trip.
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  int x = (int)v;
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);  // row_shr:1 (0 at the row's start)
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(x, 15), r1 = __builtin_amdgcn_readlane(x, 31);
  const int r2 = __builtin_amdgcn_readlane(x, 47);
  const int row = lane_id() >> 4;
  x += (row > 0 ? r0 : 0) + (row > 1 ? r1 : 0) + (row > 2 ? r2 : 0);
  return (T)x;
}

// Exclusive prefix of v over the wave and the wave's total.
__device__ __forceinline__ int wave_exscan_i32(int v, int& total) {
  const int incl = wave_incl_scan(v);
  total = __builtin_amdgcn_readlane(incl, kWave - 1);
  return incl - v;
}

template <typename T>
__device__ __forceinline__ T add_in_order(T a, T b) {
#pragma clang fp contract(off)
  return a + b;
}
template <>
__device__ __forceinline__ int32_t add_in_order<int32_t>(int32_t a, int32_t b) {
  return (int32_t)((uint32_t)a + (uint32_t)b);  // wrapping, as the reference's int32 adds
}

// Exclusive prefix of v over the threads of the workgroup, in thread order;
// total = the sum over all.  Every thread must call it.
template <int NW>
__device__ __forceinline__ int block_exscan(int v, int* red, int& total) {
  const int l = lane_id(), w = threadIdx.x / kWave;
  const int incl = wave_incl_scan(v);
  __syncthreads();
  if (l == kWave - 1) red[w] = incl;
  __syncthreads();
  int pre = 0;
  total = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const int r = red[i];
    pre += i < w ? r : 0;
    total += r;
  }
  return pre + incl - v;
}

template <int NW>
__device__ __forceinline__ int block_sum(int v, int* red) {
  v = wave_sum_i(v);
  __syncthreads();
  if (lane_id() == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) t += red[i];
  return t;
}

// Hillis-Steele inclusive scan of one 128-position tile (p = h * 64 + lane).
template <typename T>
__device__ __forceinline__ void hs_scan128(T c[2], int l) {
#pragma unroll
  for (int s = 1; s < 128; s <<= 1) {
    T n[2];
    if (s < kWave) {
      const T lo0 = shfl_up_or_zero(c[0], s, l);
      const T lo1 = shfl_up_or_zero(c[1], s, l);
      // position 64 + l - s for l < s comes from register 0, lane 64 + l - s
      const int src = l - s + kWave;
      const T wrap = __builtin_bit_cast(
          T, __builtin_amdgcn_ds_bpermute((l < s ? src : l) << 2, __builtin_bit_cast(int, c[0])));
      n[0] = add_in_order(c[0], lo0);
      n[1] = add_in_order(c[1], l < s ? wrap : lo1);
    } else {  // s == 64: position p >= 64 adds position p - 64, the others add 0
      n[0] = add_in_order(c[0], (T)0);
      n[1] = add_in_order(c[1], c[0]);
    }
    c[0] = n[0];
    c[1] = n[1];
  }
}

}  // namespace tx
