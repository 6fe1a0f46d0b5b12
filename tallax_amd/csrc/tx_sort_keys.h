// Sort-key transforms shared by the row sorts (sort_rows.hip, sort_wide.hip).
//
// Reference semantics (tallax/_src/utils.py:139-200): float keys are
// standardised (NaN -> the sortable int 0x7FFFFFFE, i.e. above +inf; -0 ->
// +0) and compared as sortable ints (i < 0 ? i ^ 0x7FFFFFFF : i); bfloat16
// keys are widened to float32 first; int32 keys compare as int32.  Here the
// sortable int is further offset by 2^31 so that the order is the unsigned
// order of a u32 ("order bits").
#pragma once
#include "tx_common.h"

namespace tx {

// the 32 bits of element i of a key array: int32 and float32 as stored,
// bfloat16 widened to float32 (utils.py:144-145)
template <int DT>
__device__ __forceinline__ uint32_t key_bits_at(const void* p, int64_t i) {
  if constexpr (DT == kBF16) return ((uint32_t)((const uint16_t*)p)[i]) << 16;
  else return ((const uint32_t*)p)[i];
}

// sortable order of a key's 32 bits as an unsigned value (standardised floats)
__device__ __forceinline__ uint32_t order_from_bits(uint32_t b, int dtype) {
  if (dtype == kI32) return b ^ 0x80000000u;
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) b = 0x7FFFFFFEu;  // NaN: sortable_int_to_float(INT32_MAX - 1)
  if ((b & 0x7FFFFFFFu) == 0u) b = 0u;                   // -0 -> +0
  const int32_t s = (int32_t)b < 0 ? (int32_t)(b ^ 0x7FFFFFFFu) : (int32_t)b;
  return (uint32_t)s ^ 0x80000000u;
}

// sortable order of element i of a key array
__device__ __forceinline__ uint32_t sort_order_bits(const void* p, int dtype, int64_t i) {
  const uint32_t b = dtype == kBF16 ? key_bits_at<kBF16>(p, i) : key_bits_at<kF32>(p, i);
  return order_from_bits(b, dtype);
}

// standardised value bits back from the sortable order
__device__ __forceinline__ uint32_t order_to_value_bits(uint32_t u) {
  const int32_t s = (int32_t)(u ^ 0x80000000u);
  return s < 0 ? ((uint32_t)s ^ 0x7FFFFFFFu) : (uint32_t)s;
}

// element i of a sorted output from its order bits: int32 keys as they were,
// floats decoded (utils.py:186-195), as bfloat16 when out_dtype asks for it
__device__ __forceinline__ void store_sorted(void* out, int out_dtype, int in_dtype, int64_t i, uint32_t u) {
  if (in_dtype == kI32) {
    ((int32_t*)out)[i] = (int32_t)(u ^ 0x80000000u);
    return;
  }
  const uint32_t b = order_to_value_bits(u);
  if (out_dtype == kBF16)
    ((uint16_t*)out)[i] = (uint16_t)(b >> 16);
  else
    ((uint32_t*)out)[i] = b;
}

}  // namespace tx
