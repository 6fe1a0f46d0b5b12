// take_along_axis and cumsum for gfx950.
//
// Reference semantics:
//   * take_along_axis (tallax/_src/gather.py:11-83): out = values[idx] along
//     `axis` (0 or 1) when 0 <= idx < extent, otherwise 0 (the kernel's
//     accumulators start at 0 and only in-range indices overwrite them;
//     there is no negative wrap).
//   * cumsum (tallax/_src/cumsum.py:16-101): the array is padded with zeros
//     to (8, 128) tiles; along `axis` every tile (128 lanes for axis 1, 8
//     rows for axis 0) is scanned with Hillis-Steele steps
//     t[j] += t[j - 2^s] (all j at once), then tile i >= 1 gets the running
//     total of tiles 0..i-1, accumulated sequentially.  The tile totals are
//     the last element of each tile's scan.  reverse = the same scan on the
//     padded array flipped along `axis`.  dtype is preserved (f32: IEEE adds
//     in that order; int32: wrapping adds).
#include <stdint.h>

#include "tallax_hip.h"
#include "tx_common.h"
#include "tx_host.h"
#include "tx_scan.h"

namespace tx {

// ---------------------------------------------------------------------------
// take_along_axis
// ---------------------------------------------------------------------------

// axis 1, rows whose values fit in LDS: the row is staged once, then every
// output of the row gathers from LDS (each value byte read from HBM once).
// When the value row, the index row and the output row are 16-byte aligned and
// whole 16-byte blocks, the staging reads, the index reads and the output
// writes are 16 bytes per lane, and a thread issues all of its staging and
// index loads (kGatherBatch blocks of each) before waiting for any of them.
constexpr int kGatherNT = 256;
constexpr int kGatherBatch = 4;
template <typename T>
__global__ __launch_bounds__(kGatherNT) void gather_row_lds_kernel(const T* __restrict__ val, int64_t vcols,
                                                                   const int32_t* __restrict__ idx,
                                                                   int64_t icols, T* __restrict__ out) {
  extern __shared__ __align__(16) unsigned char smem[];
  T* row_vals = (T*)smem;
  const int64_t r = blockIdx.x;
  const int t = threadIdx.x;
  const T* vr = val + r * vcols;
  const int32_t* ir = idx + r * icols;
  T* orow = out + r * icols;
  constexpr int EPV = 16 / (int)sizeof(T);  // values per 16-byte block
  const bool vec = (((uintptr_t)vr | (uintptr_t)ir | (uintptr_t)orow) & 15u) == 0 && vcols % EPV == 0 &&
                   icols % EPV == 0;
  if (vec) {
    const uint4* v4 = (const uint4*)vr;
    const uint4* i4 = (const uint4*)ir;
    const int64_t nv = vcols / EPV;  // value blocks
    const int64_t ni = icols / 4;    // index blocks (4 indices each)
    // the first batch of index loads is issued before the staging loads
    uint4 iv[kGatherBatch];
#pragma unroll
    for (int u = 0; u < kGatherBatch; ++u) {
      const int64_t b = (int64_t)u * kGatherNT + t;
      if (b < ni) iv[u] = load_once(i4 + b);
    }
    for (int64_t b0 = 0; b0 < nv; b0 += (int64_t)kGatherBatch * kGatherNT) {
      uint4 sv[kGatherBatch];
#pragma unroll
      for (int u = 0; u < kGatherBatch; ++u) {
        const int64_t b = b0 + (int64_t)u * kGatherNT + t;
        if (b < nv) sv[u] = load_once(v4 + b);
      }
#pragma unroll
      for (int u = 0; u < kGatherBatch; ++u) {
        const int64_t b = b0 + (int64_t)u * kGatherNT + t;
        if (b < nv) ((uint4*)row_vals)[b] = sv[u];
      }
    }
    __syncthreads();
    for (int64_t ib = 0; ib < ni; ib += (int64_t)kGatherBatch * kGatherNT) {
      if (ib > 0) {
#pragma unroll
        for (int u = 0; u < kGatherBatch; ++u) {
          const int64_t b = ib + (int64_t)u * kGatherNT + t;
          if (b < ni) iv[u] = load_once(i4 + b);
        }
      }
#pragma unroll
      for (int u = 0; u < kGatherBatch; ++u) {
        const int64_t b = ib + (int64_t)u * kGatherNT + t;
        if (b >= ni) continue;
        const int32_t q[4] = {(int32_t)iv[u].x, (int32_t)iv[u].y, (int32_t)iv[u].z, (int32_t)iv[u].w};
        T o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (q[e] >= 0 && (int64_t)q[e] < vcols) ? row_vals[q[e]] : (T)0;
        if (sizeof(T) == 4) {
          ((uint4*)orow)[b] = make_uint4((uint32_t)o[0], (uint32_t)o[1], (uint32_t)o[2], (uint32_t)o[3]);
        } else {
          ((uint2*)orow)[b] = make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16));
        }
      }
    }
    return;
  }
  for (int64_t j = t; j < vcols; j += kGatherNT) row_vals[j] = vr[j];
  __syncthreads();
  for (int64_t j = t; j < icols; j += kGatherNT) {
    const int32_t i = ir[j];
    orow[j] = (i >= 0 && (int64_t)i < vcols) ? row_vals[i] : (T)0;
  }
}

// axis 1, long rows: direct gather from global memory.
template <typename T>
__global__ __launch_bounds__(256) void gather_row_kernel(const T* __restrict__ val, int64_t vcols,
                                                         const int32_t* __restrict__ idx, int64_t icols,
                                                         int64_t total, T* __restrict__ out) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / icols;
    const int32_t i = idx[e];
    out[e] = (i >= 0 && (int64_t)i < vcols) ? val[r * vcols + i] : (T)0;
  }
}

// axis 0: out[i, c] = val[idx[i, c], c].
template <typename T>
__global__ __launch_bounds__(256) void gather_col_kernel(const T* __restrict__ val, int64_t vrows, int64_t cols,
                                                         const int32_t* __restrict__ idx, int64_t total,
                                                         T* __restrict__ out) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t c = e % cols;
    const int32_t i = idx[e];
    out[e] = (i >= 0 && (int64_t)i < vrows) ? val[(int64_t)i * cols + c] : (T)0;
  }
}

// ---------------------------------------------------------------------------
// cumsum along axis 1: one workgroup per row, 16 waves; wave w scans tiles
// w, w + 16, ... of a chunk of up to 16 * kTPW tiles held in registers (two
// elements per lane per tile: tile position p = h * 64 + lane).
// ---------------------------------------------------------------------------
constexpr int kScanNT = 1024;
constexpr int kScanNW = kScanNT / kWave;
constexpr int kTPW = 4;                        // tiles per wave per chunk
constexpr int kChunkTiles = kScanNW * kTPW;    // 64 tiles = 8192 elements

template <typename T>
__global__ __launch_bounds__(kScanNT) void cumsum_rows_kernel(const T* __restrict__ x, int64_t cols, int reverse,
                                                              T* __restrict__ out) {
  __shared__ T tsum[kChunkTiles];   // tile totals of the chunk
  __shared__ T carry[kChunkTiles];  // running total before each tile
  __shared__ T run_sh;
  const int64_t r = blockIdx.x;
  const int w = threadIdx.x / kWave, l = lane_id();
  const int64_t pcols = (cols + 127) / 128 * 128;  // padded length
  const int64_t ntiles = pcols / 128;
  const T* xr = x + r * cols;
  T* orow = out + r * cols;
  // element at scan position q (of the possibly flipped padded row)
  auto src_index = [&](int64_t q) -> int64_t { return reverse ? pcols - 1 - q : q; };
  T run = (T)0;
  for (int64_t t0 = 0; t0 < ntiles; t0 += kChunkTiles) {
    T c[kTPW][2];
#pragma unroll
    for (int i = 0; i < kTPW; ++i) {
      const int64_t t = t0 + w + (int64_t)i * kScanNW;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t q = t * 128 + h * kWave + l;
        const int64_t e = src_index(q);
        c[i][h] = (t < ntiles && e < cols) ? xr[e] : (T)0;
      }
      hs_scan128(c[i], l);
      if (l == kWave - 1) tsum[w + i * kScanNW] = c[i][1];
    }
    __syncthreads();
    // sequential running total over the chunk's tiles (reference order)
    if (threadIdx.x == 0) {
      T acc = run;
      const int64_t n = ntiles - t0 < kChunkTiles ? ntiles - t0 : kChunkTiles;
      for (int i = 0; i < n; ++i) {
        carry[i] = acc;
        acc = (t0 + i == 0) ? tsum[i] : add_in_order(acc, tsum[i]);
      }
      run_sh = acc;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kTPW; ++i) {
      const int64_t t = t0 + w + (int64_t)i * kScanNW;
      if (t >= ntiles) continue;
      const T cy = carry[w + i * kScanNW];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t q = t * 128 + h * kWave + l;
        const int64_t e = src_index(q);
        const T v = t == 0 ? c[i][h] : add_in_order(c[i][h], cy);
        if (e < cols) orow[e] = v;
      }
    }
    run = run_sh;
    __syncthreads();
  }
}

// cumsum along axis 0: one thread per column, tiles of 8 rows.
template <typename T>
__global__ __launch_bounds__(256) void cumsum_cols_kernel(const T* __restrict__ x, int64_t rows, int64_t cols,
                                                          int reverse, T* __restrict__ out) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  const int64_t prows = (rows + 7) / 8 * 8;
  T run = (T)0;
  for (int64_t t = 0; t < prows / 8; ++t) {
    T v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t q = t * 8 + i;
      const int64_t rr = reverse ? prows - 1 - q : q;
      v[i] = rr < rows ? x[rr * cols + c] : (T)0;
    }
#pragma unroll
    for (int s = 1; s < 8; s <<= 1) {
      T n[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) n[i] = add_in_order(v[i], i >= s ? v[i - s] : (T)0);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = n[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t q = t * 8 + i;
      const int64_t rr = reverse ? prows - 1 - q : q;
      if (rr < rows) out[rr * cols + c] = t == 0 ? v[i] : add_in_order(v[i], run);
    }
    run = t == 0 ? v[7] : add_in_order(run, v[7]);
  }
}

// out[0, n) = 0 (a kernel, not a memset node, so callers may capture it)
__global__ __launch_bounds__(256) void zero_fill_kernel(uint8_t* out, int64_t n) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x)
    out[e] = 0;
}

static unsigned grid_for(int64_t total) {
  int64_t b = (total + 255) / 256;
  return (unsigned)(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

}  // namespace tx

using namespace tx;

extern "C" {

int tallax_take_along_axis(const void* values, int dtype, int64_t vrows, int64_t vcols, const int32_t* indices,
                           int64_t irows, int64_t icols, int axis, void* out, hipStream_t stream) {
  if (!values || !indices || !out) { set_error("null pointer argument"); return kInvalidArgument; }
  if (dtype != kF32 && dtype != kBF16 && dtype != kI32) { set_error("dtype %d not supported", dtype); return kUnsupported; }
  if (axis != 0 && axis != 1) { set_error("axis must be 0 or 1, got %d", axis); return kInvalidArgument; }
  if (vrows < 0 || vcols < 0 || irows < 0 || icols < 0) { set_error("negative extent"); return kInvalidArgument; }
  if (axis == 1 && vrows != irows) {
    set_error("batch extents differ: values %lld rows, indices %lld rows", (long long)vrows, (long long)irows);
    return kInvalidArgument;
  }
  if (axis == 0 && vcols != icols) {
    set_error("batch extents differ: values %lld cols, indices %lld cols", (long long)vcols, (long long)icols);
    return kInvalidArgument;
  }
  const int64_t total = irows * icols;
  if (total == 0) return kOk;
  const int es = dtype == kBF16 ? 2 : 4;
  if (axis == 1) {
    if (vcols == 0) {
      // every index is out of range
      hipLaunchKernelGGL(zero_fill_kernel, dim3(grid_for(total * es)), dim3(256), 0, stream, (uint8_t*)out,
                         total * es);
      return launch_status("tallax_take_along_axis");
    }
    if (vcols * es <= 64 * 1024 && irows <= 2147483647) {
      const size_t lds = (size_t)vcols * es;
      if (es == 2)
        hipLaunchKernelGGL(gather_row_lds_kernel<uint16_t>, dim3((unsigned)irows), dim3(kGatherNT), lds, stream,
                           (const uint16_t*)values, vcols, indices, icols, (uint16_t*)out);
      else
        hipLaunchKernelGGL(gather_row_lds_kernel<uint32_t>, dim3((unsigned)irows), dim3(kGatherNT), lds, stream,
                           (const uint32_t*)values, vcols, indices, icols, (uint32_t*)out);
    } else if (es == 2) {
      hipLaunchKernelGGL(gather_row_kernel<uint16_t>, dim3(grid_for(total)), dim3(256), 0, stream,
                         (const uint16_t*)values, vcols, indices, icols, total, (uint16_t*)out);
    } else {
      hipLaunchKernelGGL(gather_row_kernel<uint32_t>, dim3(grid_for(total)), dim3(256), 0, stream,
                         (const uint32_t*)values, vcols, indices, icols, total, (uint32_t*)out);
    }
  } else {
    if (es == 2)
      hipLaunchKernelGGL(gather_col_kernel<uint16_t>, dim3(grid_for(total)), dim3(256), 0, stream,
                         (const uint16_t*)values, vrows, icols, indices, total, (uint16_t*)out);
    else
      hipLaunchKernelGGL(gather_col_kernel<uint32_t>, dim3(grid_for(total)), dim3(256), 0, stream,
                         (const uint32_t*)values, vrows, icols, indices, total, (uint32_t*)out);
  }
  return launch_status("tallax_take_along_axis");
}

int tallax_cumsum(const void* x, int dtype, int64_t rows, int64_t cols, int axis, int reverse, void* out,
                  hipStream_t stream) {
  if (!x || !out) { set_error("null pointer argument"); return kInvalidArgument; }
  if (dtype != kF32 && dtype != kI32) {
    set_error("cumsum supports f32 and int32 (dtype %d); cast bfloat16 to f32 first", dtype);
    return kUnsupported;
  }
  if (axis != 0 && axis != 1) { set_error("axis must be 0 or 1, got %d", axis); return kInvalidArgument; }
  if (rows < 0 || cols < 0) { set_error("negative extent"); return kInvalidArgument; }
  if (rows == 0 || cols == 0) return kOk;
  if (axis == 1) {
    if (rows > 2147483647) { set_error("too many rows"); return kUnsupported; }
    if (dtype == kF32)
      hipLaunchKernelGGL(cumsum_rows_kernel<float>, dim3((unsigned)rows), dim3(kScanNT), 0, stream,
                         (const float*)x, cols, reverse, (float*)out);
    else
      hipLaunchKernelGGL(cumsum_rows_kernel<int32_t>, dim3((unsigned)rows), dim3(kScanNT), 0, stream,
                         (const int32_t*)x, cols, reverse, (int32_t*)out);
  } else {
    const unsigned blocks = (unsigned)((cols + 255) / 256);
    if (dtype == kF32)
      hipLaunchKernelGGL(cumsum_cols_kernel<float>, dim3(blocks), dim3(256), 0, stream, (const float*)x, rows,
                         cols, reverse, (float*)out);
    else
      hipLaunchKernelGGL(cumsum_cols_kernel<int32_t>, dim3(blocks), dim3(256), 0, stream, (const int32_t*)x,
                         rows, cols, reverse, (int32_t*)out);
  }
  return launch_status("tallax_cumsum");
}

}  // extern "C"
