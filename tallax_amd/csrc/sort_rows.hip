// Row-wise stable sort for gfx950: the kernel under tax.sort, tumpy.sort and
// tumpy.argsort.
//
// Reference semantics (tallax/_src/sort.py:768-929, utils.py:139-227):
//   * float keys are standardised (NaN -> the sortable int 0x7FFFFFFE, i.e.
//     above +inf; -0 -> +0) and compared as sortable ints
//     (i < 0 ? i ^ 0x7FFFFFFF : i); bfloat16 keys are widened to float32
//     first; int32 keys compare as int32.  Sorted float keys come back
//     decoded from the sortable ints (so -0 -> +0 and NaN -> 0x7FFFFFFE),
//     as float32 for bfloat16 keys on the unpacked path and as bfloat16 on
//     the packed bf16+index path (NaN -> 0x7FFF there).
//   * a stable sort orders ties by ascending original index in both
//     directions (sort.py:804-813, 925-926); the packed bf16 path with a
//     non-stable descending argsort orders ties by descending index (the
//     packed key makes the order unique, utils.py:205-216).
//
// Four kernels, by row length:
//   * rows of at most 32 elements: one thread per row, a register bitonic
//     network over the same records (sort_narrow_rows_kernel);
//   * one workgroup per row from here on.  Rows of at most 512 elements: records (transformed key, tie value) are
//     padded to P = 2^m >= cols with the largest record and sorted ascending
//     by a bitonic network (sort_rows_kernel, P / 4 threads).  Each thread
//     holds E consecutive records in registers; strides < E are exchanged
//     within the thread, strides < 64 E across lanes with DPP /
//     v_permlane*_swap, larger strides through LDS;
//   * packed bf16 rows of 2049-4096 elements, at most 256 rows: a stable LSD
//     radix sort of 32-bit records (radix_sort_rows_kernel, two passes of
//     8-bit digits, 1024 threads);
//   * everything else up to 16384 elements: the wide sort's chunk radix sort
//     run on the whole row (sort_row_radix_kernel, sort_wide.hip).  The
//     bitonic network's LDS traffic grows as n log^2 n: at [256, 16384] f32
//     it took 190.8 us against 32.4 us for the radix sort, at [256, 2048]
//     12.1 against 7.5, at [1024, 1024] 14.6 against 12.4; at [1024, 256]
//     the network is faster (6.2 against 9.1 us), and the 1024-thread
//     packed radix sort wins only at config 2's shape (7.8 against 9.0 us at
//     [256, 4096] bf16; 23.9 against 19.6 at [1024, 3000]).
#include <stdint.h>

#include "tallax_hip.h"
#include "tx_common.h"
#include "tx_host.h"
#include "tx_block_sort.h"
#include "tx_scan.h"
#include "tx_sort_keys.h"
#include "tx_wave_sort.h"

namespace tx {

constexpr int kSortMaxCols = 16384;
constexpr int kSortNarrowCols = 32;  // rows sorted by one thread each

template <typename R>
struct RecT;
template <>
struct RecT<uint64_t> {  // key << 32 | tie (tie < 2^31)
  static constexpr int kTieBits = 32;
  __device__ static uint64_t make(uint32_t key, uint32_t tie) { return ((uint64_t)key << 32) | tie; }
  __device__ static uint32_t key(uint64_t r) { return (uint32_t)(r >> 32); }
  __device__ static uint32_t tie(uint64_t r) { return (uint32_t)r; }
};
template <>
struct RecT<uint32_t> {  // bf16 keys: (key >> 16) << 16 | tie (tie < 2^16)
  static constexpr int kTieBits = 16;
  __device__ static uint32_t make(uint32_t key, uint32_t tie) { return (key & 0xFFFF0000u) | tie; }
  __device__ static uint32_t key(uint32_t r) { return r & 0xFFFF0000u; }
  __device__ static uint32_t tie(uint32_t r) { return r & 0xFFFFu; }
};

template <typename R, int E, int P>
__global__ __launch_bounds__(P / E) void sort_rows_kernel(SortArgs a) {
  using RT = RecT<R>;
  extern __shared__ __align__(16) unsigned char smem[];
  R* lds = (R*)smem;
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t base = row * a.cols;
  const uint32_t tie_mask = RT::kTieBits == 32 ? 0x7FFFFFFFu : 0xFFFFu;
  R v[E];
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int i = t * E + r;
    if (i < a.cols) {
      const int64_t src = a.perm_in ? (int64_t)a.perm_in[base + i] : (int64_t)i;
      uint32_t k = sort_order_bits(a.key, a.key_dtype, base + src);
      if (a.descending) k = ~k;
      const uint32_t tie = a.ties_desc ? (tie_mask - (uint32_t)i) : (uint32_t)i;
      v[r] = RT::make(k, tie);
    } else {
      v[r] = ~(R)0;  // padding: after every real record
    }
  }
  block_bitonic_sort_c<R, E, P, false>(v, lds);
  // outputs
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int i = t * E + r;
    if (i >= a.cols) continue;
    const uint32_t tie = RT::tie(v[r]);
    const int pos = a.ties_desc ? (int)(tie_mask - tie) : (int)tie;
    const int32_t src = a.perm_in ? a.perm_in[base + pos] : pos;
    a.perm_out[base + i] = src;
    if (a.key_out) {
      uint32_t k = RT::key(v[r]);
      if (a.descending) k = ~k;
      if (sizeof(R) == 4) {  // rebuild the full order bits of a bf16 key from its high half
        k &= 0xFFFF0000u;
        if (k < 0x80000000u) k |= 0xFFFFu;         // negative values: low half of the order is all ones
        else if (k > 0xFF800000u) k = 0xFFFFFFFEu;  // the NaN sentinel 0x7FFFFFFE
      }
      store_sorted(a.key_out, a.key_out_dtype, a.key_dtype, base + i, k);
    }
    if (a.aux_out) {
      const uint32_t u = sort_order_bits(a.aux, a.aux_dtype, base + src);
      store_sorted(a.aux_out, a.aux_out_dtype, a.aux_dtype, base + i, u);
    }
  }
}

constexpr int kRadixNT = 1024;

// out[i] = the key at column perm[i] of the same row, standardised and
// decoded like the sorted key outputs (store_sorted): the third and later
// keys of a multi-key sort.  A column outside the row gives 0 bits.
__global__ __launch_bounds__(256) void gather_sort_key_kernel(const void* key, int key_dtype, int64_t cols,
                                                              const int32_t* perm, void* out, int out_dtype,
                                                              int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t base = i / cols * cols;
    const int32_t src = perm[i];
    if (src >= 0 && src < cols) {
      store_sorted(out, out_dtype, key_dtype, i, sort_order_bits(key, key_dtype, base + src));
    } else if (out_dtype == kBF16) {
      ((uint16_t*)out)[i] = 0;
    } else {
      ((uint32_t*)out)[i] = 0u;
    }
  }
}

// bf16 keys (records of a 16-bit key and a 16-bit tie): a stable LSD radix
// sort on the key, two passes of 8-bit digits.  The records start in
// ascending tie order (slot p holds tie p), so sorting by key alone, stably,
// is the ascending record order the bitonic network gives.  The 4096 record
// slots of a row sit record-major inside each wave: slot p = 256 w + 64 r + l
// is record r of lane l of wave w, so the wave's slots in ascending order are
// (r, l).  Per pass:
//   * each wave counts its digits in its own 256 counters (digit-major, 17
//     words apart, so that random digits spread over the banks) with one LDS
//     atomic per record, record r = 0..3 in turn.  The atomics of one
//     instruction on one address return in ascending lane order (gfx950), so
//     the value before a record's increment is its rank among the wave's
//     earlier slots of that digit: a stable rank;
//   * an exclusive scan over (digit, wave) in digit-major order gives each
//     pair its start, and records move to start + rank through LDS;
//   * slots past the row hold all-ones records, which every pass keeps after
//     the row's own (their slots are the highest, their digits the largest).
// (Four passes of 4-bit digits with per-thread packed counters took 13.0 us at
// config 2; these two passes, with the same three barriers each, 1.6 us less.)
template <int BITS>
__global__ __launch_bounds__(kRadixNT) void radix_sort_rows_kernel(SortArgs a) {
  static_assert(BITS == 8, "8-bit digits: 256 counters per wave");
  using RT = RecT<uint32_t>;
  constexpr int NW = kRadixNT / kWave;  // 16 waves, 256 slots each
  constexpr int HS = NW + 1;            // counter stride per digit
  __shared__ uint32_t hist[256 * HS];
  __shared__ uint32_t buf[4 * kRadixNT];
  __shared__ uint32_t wsum[NW];
  const int t = threadIdx.x, l = lane_id(), w = t / kWave;
  const int n = (int)a.cols;
  const int64_t row = blockIdx.x;
  const int64_t base = row * a.cols;
  uint32_t v[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int p = w * 256 + r * kWave + l;
    v[r] = ~0u;
    if (p < n) {
      const int i = a.ties_desc ? n - 1 - p : p;  // ascending ties either way
      uint32_t k = sort_order_bits(a.key, a.key_dtype, base + i);
      if (a.descending) k = ~k;
      v[r] = RT::make(k, a.ties_desc ? 0xFFFFu - (uint32_t)i : (uint32_t)i);
    }
  }
#pragma unroll 1
  for (int sh = 16; sh < 32; sh += 8) {
#pragma unroll
    for (int d = l; d < 256; d += kWave) hist[d * HS + w] = 0u;  // this wave's counters
    uint32_t dg[4], rk[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      dg[r] = (v[r] >> sh) & 0xFFu;
      rk[r] = atomicAdd(&hist[dg[r] * HS + w], 1u);
    }
    __syncthreads();  // every count is in
    // exclusive scan over i = digit * NW + wave: thread t takes i = 4t .. 4t + 3
    const int d0 = t >> 2, w0 = 4 * (t & 3);
    uint32_t c[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) c[q] = hist[d0 * HS + w0 + q];
    const uint32_t run = c[0] + c[1] + c[2] + c[3];
    const uint32_t incl = wave_incl_scan(run);
    if (l == kWave - 1) wsum[w] = incl;
    __syncthreads();
    uint32_t pre = incl - run;
#pragma unroll
    for (int i = 0; i < NW; ++i) pre += i < w ? wsum[i] : 0u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      hist[d0 * HS + w0 + q] = pre;
      pre += c[q];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; ++r) buf[hist[dg[r] * HS + w] + rk[r]] = v[r];
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = buf[w * 256 + r * kWave + l];
  }
  const uint32_t tie_mask = 0xFFFFu;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = w * 256 + r * kWave + l;
    if (i >= n) continue;
    const uint32_t tie = RT::tie(v[r]);
    const int pos = a.ties_desc ? (int)(tie_mask - tie) : (int)tie;
    a.perm_out[base + i] = pos;
    if (a.key_out) {
      uint32_t k = RT::key(v[r]);
      if (a.descending) k = ~k;
      k &= 0xFFFF0000u;  // rebuild the full order bits of a bf16 key from its high half
      if (k < 0x80000000u) k |= 0xFFFFu;
      else if (k > 0xFF800000u) k = 0xFFFFFFFEu;
      store_sorted(a.key_out, a.key_out_dtype, a.key_dtype, base + i, k);
    }
    if (a.aux_out) {
      const uint32_t u = sort_order_bits(a.aux, a.aux_dtype, base + pos);
      store_sorted(a.aux_out, a.aux_out_dtype, a.aux_dtype, base + i, u);
    }
  }
}

// Rows of at most NC (16 or 32) elements: one thread per row, the row's
// records sorted in registers by a bitonic network (ascending records; the
// padding records, all ones, go last), then the same outputs as
// sort_rows_kernel.  A wave per row would spend 256 padded slots on 8
// elements ([1000000, 8] f32 argsort: 1154 us that way).
template <typename R, int NC>
__global__ __launch_bounds__(256) void sort_narrow_rows_kernel(SortArgs a, int64_t rows) {
  using RT = RecT<R>;
  const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  const int64_t base = row * a.cols;
  const int cols = (int)a.cols;
  const uint32_t tie_mask = RT::kTieBits == 32 ? 0x7FFFFFFFu : 0xFFFFu;
  R v[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    if (i < cols) {
      const int64_t src = a.perm_in ? (int64_t)a.perm_in[base + i] : (int64_t)i;
      uint32_t k = sort_order_bits(a.key, a.key_dtype, base + src);
      if (a.descending) k = ~k;
      const uint32_t tie = a.ties_desc ? (tie_mask - (uint32_t)i) : (uint32_t)i;
      v[i] = RT::make(k, tie);
    } else {
      v[i] = ~(R)0;
    }
  }
#pragma unroll
  for (int k = 2; k <= NC; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const int o = i ^ j;
        if (o > i) {
          const R x = v[i], y = v[o];
          const bool up = (i & k) == 0;  // this block ascends
          const bool sw = up ? x > y : x < y;
          v[i] = sw ? y : x;
          v[o] = sw ? x : y;
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    if (i >= cols) continue;
    const uint32_t tie = RT::tie(v[i]);
    const int pos = a.ties_desc ? (int)(tie_mask - tie) : (int)tie;
    const int32_t src = a.perm_in ? a.perm_in[base + pos] : pos;
    a.perm_out[base + i] = src;
    if (a.key_out) {
      uint32_t k = RT::key(v[i]);
      if (a.descending) k = ~k;
      if (sizeof(R) == 4) {  // rebuild the full order bits of a bf16 key from its high half
        k &= 0xFFFF0000u;
        if (k < 0x80000000u) k |= 0xFFFFu;
        else if (k > 0xFF800000u) k = 0xFFFFFFFEu;
      }
      store_sorted(a.key_out, a.key_out_dtype, a.key_dtype, base + i, k);
    }
    if (a.aux_out) {
      const uint32_t u = sort_order_bits(a.aux, a.aux_dtype, base + src);
      store_sorted(a.aux_out, a.aux_out_dtype, a.aux_dtype, base + i, u);
    }
  }
}

template <typename R>
static int launch_sort_narrow(const SortArgs& a, int64_t rows, hipStream_t s) {
  const unsigned grid = (unsigned)((rows + 255) / 256);
  if (a.cols <= 16)
    hipLaunchKernelGGL((sort_narrow_rows_kernel<R, 16>), dim3(grid), dim3(256), 0, s, a, rows);
  else
    hipLaunchKernelGGL((sort_narrow_rows_kernel<R, 32>), dim3(grid), dim3(256), 0, s, a, rows);
  return kOk;
}

static int launch_radix8(const SortArgs& a, int64_t rows, hipStream_t s) {
  hipLaunchKernelGGL((radix_sort_rows_kernel<8>), dim3((unsigned)rows), dim3(kRadixNT), 0, s, a);
  return kOk;
}

template <typename R, int E, int P>
static int launch_sort(const SortArgs& a, int64_t rows, hipStream_t s) {
  const size_t lds = (size_t)P * sizeof(R);
  if (lds > 64 * 1024) {
    const hipError_t attr = set_dynamic_lds_limit((const void*)sort_rows_kernel<R, E, P>, (int)lds, s);
    if (attr != hipSuccess) {
      set_error("hipFuncSetAttribute: %s", hipGetErrorString(attr));
      return kHipError;
    }
  }
  hipLaunchKernelGGL((sort_rows_kernel<R, E, P>), dim3((unsigned)rows), dim3(P / E), lds, s, a);
  return kOk;
}

template <typename R>
static int launch_sort_p(const SortArgs& a, int64_t rows, hipStream_t s) {  // rows of at most 512 elements
  return a.P == 256 ? launch_sort<R, 4, 256>(a, rows, s) : launch_sort<R, 4, 512>(a, rows, s);
}

}  // namespace tx

using namespace tx;

extern "C" {

size_t tallax_sort_rows_workspace_size(int64_t rows, int64_t cols) {
  return sort_wide_workspace_bytes(rows, cols);
}

int tallax_sort_rows_ws(const void* key, int key_dtype, int64_t rows, int64_t cols, int descending,
                        int ties_descending, const int32_t* perm_in, int32_t* perm_out, void* key_out,
                        int key_out_dtype, const void* aux, int aux_dtype, void* aux_out, int aux_out_dtype,
                        void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!key || !perm_out) { set_error("null pointer argument"); return kInvalidArgument; }
  for (int d : {key_dtype, aux ? aux_dtype : kF32}) {
    if (d != kF32 && d != kBF16 && d != kI32) { set_error("dtype %d not supported", d); return kUnsupported; }
  }
  if ((aux == nullptr) != (aux_out == nullptr)) { set_error("aux and aux_out go together"); return kInvalidArgument; }
  auto out_ok = [](int in, int out) {
    return in == kBF16 ? (out == kBF16 || out == kF32) : out == in;
  };
  if (key_out && !out_ok(key_dtype, key_out_dtype)) { set_error("key_out dtype %d invalid for key dtype %d", key_out_dtype, key_dtype); return kInvalidArgument; }
  if (aux_out && !out_ok(aux_dtype, aux_out_dtype)) { set_error("aux_out dtype %d invalid for aux dtype %d", aux_out_dtype, aux_dtype); return kInvalidArgument; }
  if (rows < 0 || cols < 0) { set_error("negative extent"); return kInvalidArgument; }
  if (rows == 0 || cols == 0) return kOk;
  if (rows > 2147483647) { set_error("too many rows"); return kUnsupported; }
  SortArgs a = {};
  a.key = key; a.key_dtype = key_dtype; a.cols = cols;
  int P = 256;
  while (P < cols && P <= kSortMaxCols) P <<= 1;  // the in-LDS network's padded length
  a.P = P;
  a.descending = descending != 0;
  a.ties_desc = ties_descending != 0;
  a.perm_in = perm_in; a.perm_out = perm_out;
  a.key_out = key_out; a.key_out_dtype = key_out_dtype;
  a.aux = aux; a.aux_dtype = aux_dtype; a.aux_out = aux_out; a.aux_out_dtype = aux_out_dtype;
  if (cols > kSortMaxCols) {  // longer than one workgroup's LDS: chunk sorts + merge passes
    const int st = launch_sort_wide(a, rows, workspace, workspace_bytes, stream);
    return st ? st : launch_status("tallax_sort_rows");
  }
  // bf16 keys on the packed path fit (16-bit key | 16-bit tie) in one u32
  const bool narrow = key_dtype == kBF16 && !perm_in && cols <= 65536;
  int st;
  if (narrow && rows <= 256 && cols > 2048 && cols <= 4 * kRadixNT)
    st = launch_radix8(a, rows, stream);
  else if (cols <= kSortNarrowCols)
    st = narrow ? launch_sort_narrow<uint32_t>(a, rows, stream) : launch_sort_narrow<uint64_t>(a, rows, stream);
  else if (cols <= 512)
    st = narrow ? launch_sort_p<uint32_t>(a, rows, stream) : launch_sort_p<uint64_t>(a, rows, stream);
  else
    st = launch_sort_row_radix(a, rows, stream);
  if (st) return st;
  return launch_status("tallax_sort_rows");
}

int tallax_gather_sort_key(const void* key, int key_dtype, int64_t rows, int64_t cols, const int32_t* perm,
                           void* out, int out_dtype, hipStream_t stream) {
  if (!key || !perm || !out) { set_error("null pointer argument"); return kInvalidArgument; }
  if (key_dtype != kF32 && key_dtype != kBF16 && key_dtype != kI32) { set_error("dtype %d not supported", key_dtype); return kUnsupported; }
  const bool ok = key_dtype == kBF16 ? (out_dtype == kBF16 || out_dtype == kF32) : out_dtype == key_dtype;
  if (!ok) { set_error("out dtype %d invalid for key dtype %d", out_dtype, key_dtype); return kInvalidArgument; }
  if (rows < 0 || cols < 0) { set_error("negative extent"); return kInvalidArgument; }
  const int64_t n = rows * cols;
  if (n == 0) return kOk;
  const int64_t blocks = (n + 255) / 256 < ((int64_t)1 << 20) ? (n + 255) / 256 : ((int64_t)1 << 20);
  hipLaunchKernelGGL(gather_sort_key_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, key, key_dtype, cols,
                     perm, out, out_dtype, n);
  return launch_status("tallax_gather_sort_key");
}

int tallax_sort_rows(const void* key, int key_dtype, int64_t rows, int64_t cols, int descending,
                     int ties_descending, const int32_t* perm_in, int32_t* perm_out, void* key_out,
                     int key_out_dtype, const void* aux, int aux_dtype, void* aux_out, int aux_out_dtype,
                     hipStream_t stream) {
  return tallax_sort_rows_ws(key, key_dtype, rows, cols, descending, ties_descending, perm_in, perm_out, key_out,
                             key_out_dtype, aux, aux_dtype, aux_out, aux_out_dtype, nullptr, 0, stream);
}

}  // extern "C"
