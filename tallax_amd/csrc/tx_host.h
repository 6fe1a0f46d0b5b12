// Host-side helpers shared by the C-ABI entry points.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

namespace tx {

enum Status : int {
  kOk = 0,
  kInvalidArgument = 1,   // shapes / sizes / pointers the op rejects
  kUnsupported = 2,       // valid request this build does not implement
  kHipError = 3,          // the HIP runtime reported an error at launch
  kWorkspaceTooSmall = 4,
};

// Thread-local message read back by tallax_last_error().
void set_error(const char* fmt, ...);

inline int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: HIP launch failed: %s", what, hipGetErrorString(e));
    return kHipError;
  }
  return kOk;
}

// float -> nearest bfloat16 (ties to even; NaN stays NaN), as a float
inline float round_to_bf16(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  if ((b & 0x7fffffffu) > 0x7f800000u) {
    b = (b | 0x00400000u) & 0xffff0000u;
  } else {
    b = (b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u;
  }
  float r;
  memcpy(&r, &b, 4);
  return r;
}

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Raise a kernel's dynamic-LDS limit to `bytes` on the device of `stream`
// (the current device for the null stream).  The attribute is per device;
// each (device, kernel) pair is set once.
hipError_t set_dynamic_lds_limit(const void* kernel, int bytes, hipStream_t stream);

// Per-segment sorted top-128 composites of every row (row_select.hip):
// plan the segments (at least min_seg per row), then launch the segment kernel
// writing lists[rows][nseg][128].
int segment_lists_plan(int64_t rows, int64_t cols, int dt, int min_seg, int* nseg_out, int* maxv_out,
                       int64_t* vps_out);
int launch_segment_lists(const void* x, int dt, int64_t rows, int64_t cols, int nseg, int maxv, int64_t vps,
                         uint64_t* lists, hipStream_t s);

// Arguments of a row sort (sort_rows.hip, sort_wide.hip).
struct SortArgs {
  const void* key;
  int key_dtype;
  int64_t cols;
  int P;            // padded length, power of two (in-LDS sorts)
  int descending;
  int ties_desc;    // ties by descending original index
  const int32_t* perm_in;  // optional: sort key[perm_in] with position ties, compose
  int32_t* perm_out;
  void* key_out;
  int key_out_dtype;
  const void* aux;  // optional second key, output gathered by the final permutation
  int aux_dtype;
  void* aux_out;
  int aux_out_dtype;
};

// Rows longer than one workgroup's LDS holds (sort_wide.hip): chunk sorts and
// merge passes through a workspace of sort_wide_workspace_bytes bytes.
size_t sort_wide_workspace_bytes(int64_t rows, int64_t cols);
int launch_sort_wide(const SortArgs& a, int64_t rows, void* ws, size_t ws_bytes, hipStream_t s);
// Rows of at most 16384 elements sorted whole by one workgroup each with the
// chunk pass's LSD radix sort (sort_wide.hip).
int launch_sort_row_radix(const SortArgs& a, int64_t rows, hipStream_t s);

}  // namespace tx
