// Shared device helpers for the tallax MI355X (gfx950) kernels.
//
// Everything here is wave64 CDNA4 code: cross-lane traffic uses VALU lane
// exchanges (DPP and gfx950's v_permlane16/32_swap) rather than LDS-unit
// shuffles, and no kernel uses MFMA (nothing on the sort / select / sample
// path is a dense contraction).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tx {

constexpr int kWave = 64;

enum DType : int { kF32 = 0, kBF16 = 1, kI32 = 2 };

// ---------------------------------------------------------------------------
// Selection keys.
//
// A "select key" orders numbers the way the reference's top-k does: values
// are compared as floats with strict `>` (tallax/_src/top_k.py:64), so -0 and
// +0 are equal and NaN never wins a comparison.  We map a float's bits to an
// unsigned 32-bit key that is monotone in value, with +0 == -0, and NaN mapped
// to 1 (below -inf).  Key 0 is reserved for "no element" (out-of-row slots).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t select_key(uint32_t b) {
  const uint32_t a = b & 0x7FFFFFFFu;
  uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  k = (a == 0u) ? 0x80000000u : k;
  k = (a > 0x7F800000u) ? 1u : k;
  return k;
}

// Inverse of select_key for keys of real numbers (keys >= 0x007FFFFF).
__device__ __forceinline__ uint32_t key_to_bits(uint32_t k) {
  return (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
}

// Keys at or below this value belong to elements the reference's binned
// top-k can never select: its bins start at finfo(dtype).min and only admit
// strictly greater values (top_k.py:241-243, :64).  That excludes -inf, NaN
// and finfo.min itself.  For f32 the key of -FLT_MAX is 0x00800000; bf16's
// finfo.min (0xFF7F) widens to 0xFF7F0000 whose key is 0x0080FFFF.
__device__ __forceinline__ uint32_t ineligible_key_max(int dt) {
  return dt == kBF16 ? 0x0080FFFFu : 0x00800000u;
}

// Composite key: value descending, then index ascending, as one u64 so that
// every element of a row has a distinct key and "larger composite" == "earlier
// in the lowest-index-tie-break order".
__device__ __forceinline__ uint64_t make_comp(uint32_t key, uint32_t idx) {
  return ((uint64_t)key << 32) | (uint64_t)(~idx);
}
__device__ __forceinline__ uint32_t comp_key(uint64_t c) { return (uint32_t)(c >> 32); }
__device__ __forceinline__ int32_t comp_idx(uint64_t c) { return (int32_t)(~(uint32_t)c); }

// ---------------------------------------------------------------------------
// Wave helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

// 16-byte load of data that is read once: the nontemporal hint streams it
// past the caches instead of evicting what stays resident there (the
// kernel's code, the small arrays every workgroup reads).
__device__ __forceinline__ uint4 load_once(const uint4* p) {
  typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
  const u32x4_nt x = __builtin_nontemporal_load((const u32x4_nt*)p);
  return make_uint4(x.x, x.y, x.z, x.w);
}

__device__ __forceinline__ uint2 load_once(const uint2* p) {
  typedef unsigned int u32x2_nt __attribute__((ext_vector_type(2)));
  const u32x2_nt x = __builtin_nontemporal_load((const u32x2_nt*)p);
  return make_uint2(x.x, x.y);
}

// s_barrier after this wave's LDS operations only: unlike __syncthreads it
// does not wait for the wave's global loads and stores to complete, which
// stay in flight across it
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// v_max_f32 / v_max3_f32 on the operands as they are.  fmaxf makes the
// compiler quiet every operand first (one v_max_f32 x, x each, since the
// hardware returns NaN for a signalling NaN); these skip that.  A quiet NaN
// operand is ignored, a signalling NaN may give NaN: use them where any NaN
// in the data already makes the result NaN.
__device__ __forceinline__ float raw_max(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float raw_max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Value of lane (lane ^ d) for d in {1, 2, 4, 8, 16, 32}, with VALU lane
// exchanges only (no LDS-unit round trip):
//   d = 1, 2   DPP quad_perm [1,0,3,2] / [2,3,0,1];
//   d = 4      DPP row_ror:12 (lane i reads i+4) or row_ror:4 (reads i-4),
//              chosen by bit 2 of the lane;
//   d = 8      DPP row_ror:8;
//   d = 16, 32 v_permlane16_swap / v_permlane32_swap of the register with
//              itself: result [0] holds the even rows (halves), [1] the odd
//              ones, so the partner is [0] on odd and [1] on even lanes.
// `d` must fold to a constant after unrolling.
__device__ __forceinline__ uint32_t lane_xor(uint32_t x, int d) {
  const int l = (int)(threadIdx.x & (kWave - 1));
  switch (d) {
    case 1: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false);
    case 2: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false);
    case 4: {
      const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x12C, 0xF, 0xF, false);
      const uint32_t dn = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x124, 0xF, 0xF, false);
      return (l & 4) ? dn : up;
    }
    case 8: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xF, 0xF, false);
    case 16: {
      const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
      return (l & 16) ? r[0] : r[1];
    }
    default: {
      const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
      return (l & 32) ? r[0] : r[1];
    }
  }
}

__device__ __forceinline__ float lane_xor_f(float x, int d) {
  return __uint_as_float(lane_xor(__float_as_uint(x), d));
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = lane_xor((uint32_t)v, m);
  const uint32_t hi = lane_xor((uint32_t)(v >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}

// Value of lane (lane - d) within a 16-lane row (DPP row_shr:d); lanes whose
// source falls outside the row read 0.  d in {1, 2, 4}, constant after unrolling.
__device__ __forceinline__ float row_shr_f(float x, int d) {
  const int v = __float_as_int(x);
  switch (d) {
    case 1: return __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true));
    case 2: return __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true));
    default: return __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true));
  }
}

// Uniform broadcast of lane `src` (src must be wave-uniform).
__device__ __forceinline__ uint32_t readlane_u32(uint32_t x, int src) {
  return (uint32_t)__builtin_amdgcn_readlane((int)x, src);
}
__device__ __forceinline__ float readlane_f(float x, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), src));
}

// Value of lane (63 - lane): DPP row_mirror reverses each 16-lane row, then
// rows are swapped pairwise (xor 16, then xor 32).
__device__ __forceinline__ uint32_t lane_rev(uint32_t x) {
  const uint32_t m = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x140, 0xF, 0xF, false);
  return lane_xor(lane_xor(m, 16), 32);
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) v += (int)lane_xor((uint32_t)v, d);
  return v;
}

// Wave maximum, written out step by step: a loop over the distances is not
// always unrolled, and lane_xor needs constant distances.
__device__ __forceinline__ int wave_max_i(int v) {
  v = max(v, (int)lane_xor((uint32_t)v, 32));
  v = max(v, (int)lane_xor((uint32_t)v, 16));
  v = max(v, (int)lane_xor((uint32_t)v, 8));
  v = max(v, (int)lane_xor((uint32_t)v, 4));
  v = max(v, (int)lane_xor((uint32_t)v, 2));
  return max(v, (int)lane_xor((uint32_t)v, 1));
}

__device__ __forceinline__ uint32_t wave_and_u32(uint32_t v) {
  v &= lane_xor(v, 32);
  v &= lane_xor(v, 16);
  v &= lane_xor(v, 8);
  v &= lane_xor(v, 4);
  v &= lane_xor(v, 2);
  return v & lane_xor(v, 1);
}
__device__ __forceinline__ uint32_t wave_or_u32(uint32_t v) {
  v |= lane_xor(v, 32);
  v |= lane_xor(v, 16);
  v |= lane_xor(v, 8);
  v |= lane_xor(v, 4);
  v |= lane_xor(v, 2);
  return v | lane_xor(v, 1);
}

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) v += lane_xor_f(v, d);
  return v;
}

// Unaligned-safe 16-byte vector source for a row.  Rows need not start on a
// 16-byte boundary: we read whole 16-byte blocks starting at the aligned-down
// address and mask out the elements that fall outside the row.  A 16-byte
// block that contains at least one byte of the row lies inside the same GPU
// page as that byte, so these reads never touch an unmapped page.
template <int ES>
struct RowVec {
  const uint4* base;  // aligned-down start
  int mis;            // number of leading elements of the first block outside the row
  __device__ __forceinline__ RowVec(const void* row_ptr) {
    const uint32_t off = (uint32_t)(uintptr_t)row_ptr & 15u;
    // pointer arithmetic (not an integer round trip) keeps the pointer's
    // provenance, so loads through it compile to global_load, not flat_load
    base = (const uint4*)((const char*)row_ptr - off);
    mis = (int)(off / ES);
  }
};

// Bit reversal of the low `bits` bits of x.
__device__ __forceinline__ uint32_t bitrev(uint32_t x, int bits) {
  return __brev(x) >> (32 - bits);
}

}  // namespace tx
