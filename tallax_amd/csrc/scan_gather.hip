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
// Value rows staged in LDS: up to 64 KiB, or 80 KiB (two workgroups per CU)
// from 512 rows.  Longer rows gather in XCD-ordered chunks instead (measured,
// f32: [64, 40960] 12.6 against 24.9 us staged, [256, 32768] 33.4 against
// 38.7, [256, 40960] 42.4 against 48.6; [512, 20000] 29.9 staged against 40.9).
constexpr int64_t kGatherLdsMax = 64 * 1024;
constexpr int64_t kGatherLdsMaxMany = 80 * 1024;
constexpr int64_t kGatherManyRows = 512;
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

// axis 1, rows longer than LDS: workgroup b runs on XCD b % 8 (dispatch
// order), and the workgroups of one XCD take the chunks of rows xcd, xcd + 8,
// ... one row after another, so the rows an XCD gathers from at a time stay
// in its own L2 (about 64 chunks per row keep ~4 rows of 0.5 MiB in flight
// per XCD).  Each thread issues kXcdBatch index loads, then the value loads
// they address, then the stores.
constexpr int kXcdBatch = 8;
template <typename T>
__global__ __launch_bounds__(256) void gather_row_xcd_kernel(const T* __restrict__ val, int64_t vcols,
                                                             const int32_t* __restrict__ idx, int64_t icols,
                                                             int64_t rows, int64_t chunks, T* __restrict__ out) {
  const int64_t b = blockIdx.x;
  const int64_t xcd = b % 8, i = b / 8;
  const int64_t r = xcd + 8 * (i / chunks);
  if (r >= rows) return;
  const int64_t ch = i % chunks;
  const int64_t per = (icols + chunks - 1) / chunks;
  const int64_t c0 = ch * per, c1 = c0 + per < icols ? c0 + per : icols;
  const T* vr = val + r * vcols;
  const int32_t* ir = idx + r * icols;
  T* orow = out + r * icols;
  for (int64_t j0 = c0 + threadIdx.x; j0 < c1; j0 += (int64_t)256 * kXcdBatch) {
    int32_t q[kXcdBatch];
#pragma unroll
    for (int u = 0; u < kXcdBatch; ++u) {
      const int64_t j = j0 + (int64_t)u * 256;
      q[u] = j < c1 ? ir[j] : -1;
    }
    T v[kXcdBatch];
#pragma unroll
    for (int u = 0; u < kXcdBatch; ++u) v[u] = (q[u] >= 0 && (int64_t)q[u] < vcols) ? vr[q[u]] : (T)0;
#pragma unroll
    for (int u = 0; u < kXcdBatch; ++u) {
      const int64_t j = j0 + (int64_t)u * 256;
      if (j < c1) orow[j] = v[u];
    }
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
// cumsum.  Tile t of a scan line (a row for axis 1, a column for axis 0) holds
// scan positions [t * TS, (t + 1) * TS) of the zero-padded line of length
// plen = ntiles * TS (TS = 128 for axis 1, 8 for axis 0); position q is
// element q, or element plen - 1 - q when reversed.  The tile's total is its
// scanned last position; for every tile but the last that position is a real
// element (forward: TS t + TS - 1 < cols; reversed: plen - TS (t + 1) >= 0),
// and its final value, scan + carry, is the carry of the next tile:
// carry[t + 1] = add(total[t], carry[t]) in the reference's sequential order.
// Last positions sit at element index = TS - 1 (mod TS) forward and 0
// (mod TS) reversed (plen is a multiple of TS).
// ---------------------------------------------------------------------------

// element index of tile t's last scan position
__device__ __forceinline__ int64_t tile_last_pos(int64_t t, int ts, int64_t plen, int reverse) {
  return reverse ? plen - (int64_t)ts * (t + 1) : (int64_t)ts * t + ts - 1;
}

// element index where the three-launch path stages tile t's total: the line's
// leading elements with the last positions skipped (TS - 1 totals per TS
// elements), so that the totals of a line are nearly contiguous and never
// share an element with a final value.  Staged indices stay below
// TS * (ntiles - 1) <= len for t <= ntiles - 2.
__device__ __forceinline__ int64_t tile_stage_pos(int64_t t, int ts, int reverse) {
  return (int64_t)ts * (t / (ts - 1)) + (reverse ? 1 : 0) + t % (ts - 1);
}

template <typename T>
__device__ __forceinline__ T readlane_t(T v, int src) {
  return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}

// Axis 1, one workgroup per row, 16 waves; wave w scans tiles w, w + 16, ...
// of a chunk of 64 tiles held in registers (two elements per lane per tile:
// tile position p = h * 64 + lane).  The next chunk's loads are issued before
// this chunk's carries are chained, and wave 0 chains the 64 tile totals with
// readlanes (one dependent add per tile).
constexpr int kScanNT = 1024;
constexpr int kScanNW = kScanNT / kWave;
constexpr int kTPW = 4;                        // tiles per wave per chunk
constexpr int kChunkTiles = kScanNW * kTPW;    // 64 tiles = 8192 elements
static_assert(kChunkTiles == kWave, "one tile total per lane of wave 0");

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
  auto load_chunk = [&](int64_t t0, T (&c)[kTPW][2]) {
#pragma unroll
    for (int i = 0; i < kTPW; ++i) {
      const int64_t t = t0 + w + (int64_t)i * kScanNW;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t q = t * 128 + h * kWave + l;
        const int64_t e = reverse ? pcols - 1 - q : q;
        c[i][h] = (t < ntiles && e < cols) ? xr[e] : (T)0;
      }
    }
  };
  T c[kTPW][2];
  load_chunk(0, c);
  T run = (T)0;
  for (int64_t t0 = 0; t0 < ntiles; t0 += kChunkTiles) {
#pragma unroll
    for (int i = 0; i < kTPW; ++i) {
      hs_scan128(c[i], l);
      if (l == kWave - 1) tsum[w + i * kScanNW] = c[i][1];
    }
    T nx[kTPW][2];
    load_chunk(t0 + kChunkTiles, nx);
    lds_barrier();
    // sequential running total over the chunk's tiles (reference order)
    if (w == 0) {
      const T mine = t0 + l < ntiles ? tsum[l] : (T)0;
      T acc = t0 == 0 ? readlane_t(mine, 0) : add_in_order(run, readlane_t(mine, 0));
      T cy = run;
#pragma unroll
      for (int i = 1; i < kChunkTiles; ++i) {
        cy = l == i ? acc : cy;
        acc = add_in_order(acc, readlane_t(mine, i));
      }
      carry[l] = cy;
      if (l == 0) run_sh = acc;
    }
    lds_barrier();
#pragma unroll
    for (int i = 0; i < kTPW; ++i) {
      const int64_t t = t0 + w + (int64_t)i * kScanNW;
      if (t >= ntiles) continue;
      const T cy = carry[w + i * kScanNW];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t q = t * 128 + h * kWave + l;
        const int64_t e = reverse ? pcols - 1 - q : q;
        const T v = t == 0 ? c[i][h] : add_in_order(c[i][h], cy);
        if (e < cols) orow[e] = v;
      }
    }
    run = run_sh;
#pragma unroll
    for (int i = 0; i < kTPW; ++i) {
      c[i][0] = nx[i][0];
      c[i][1] = nx[i][1];
    }
    // no third barrier: the next writes of tsum, carry and run_sh follow the
    // next chunk's first barrier, which every wave reaches after its reads
  }
}

// Axis 1, any number of rows, in three launches (each tile scanned by one
// wave, so the chip fills whatever the row count):
//   FINAL = false: scan tiles 0 .. ntiles - 2 of every row and stage each
//                  tile's total in `out` (tile_stage_pos);
//   cumsum_chain_kernel: chain the staged totals and store the final values
//                  at the tiles' last positions;
//   FINAL = true:  scan every tile again and add the carry (the previous
//                  tile's final last position); positions already final are
//                  not written, staged totals are overwritten.
constexpr int kTileWaves = 4;      // waves per workgroup
constexpr int kTilesPerWave = 4;   // tiles per wave, loads issued together
template <typename T, bool FINAL>
__global__ __launch_bounds__(kTileWaves * kWave) void cumsum_row_tiles_kernel(const T* __restrict__ x, int64_t rows,
                                                                              int64_t cols, int64_t ntiles,
                                                                              int reverse, T* __restrict__ out) {
  const int l = lane_id();
  const int64_t per_row = FINAL ? ntiles : ntiles - 1;
  const int64_t ntask = rows * per_row;
  const int64_t pcols = ntiles * 128;
  const int64_t g0 = ((int64_t)blockIdx.x * kTileWaves + threadIdx.x / kWave) * kTilesPerWave;
  T c[kTilesPerWave][2];
  T cy[kTilesPerWave];
  int64_t rr[kTilesPerWave], tt[kTilesPerWave];
#pragma unroll
  for (int i = 0; i < kTilesPerWave; ++i) {
    const int64_t g = g0 + i;
    rr[i] = g < ntask ? g / per_row : -1;
    tt[i] = g < ntask ? g - rr[i] * per_row : 0;
    const T* xr = x + rr[i] * cols;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t q = tt[i] * 128 + h * kWave + l;
      const int64_t e = reverse ? pcols - 1 - q : q;
      c[i][h] = (rr[i] >= 0 && e < cols) ? xr[e] : (T)0;
    }
    cy[i] = (FINAL && rr[i] >= 0 && tt[i] > 0) ? out[rr[i] * cols + tile_last_pos(tt[i] - 1, 128, pcols, reverse)]
                                               : (T)0;
  }
#pragma unroll
  for (int i = 0; i < kTilesPerWave; ++i) {
    hs_scan128(c[i], l);
    if (rr[i] < 0) continue;
    T* orow = out + rr[i] * cols;
    if (!FINAL) {
      if (l == kWave - 1) orow[tile_stage_pos(tt[i], 128, reverse)] = c[i][1];
      continue;
    }
    const bool last_final = tt[i] < ntiles - 1;  // the last position already holds its final value
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t q = tt[i] * 128 + h * kWave + l;
      const int64_t e = reverse ? pcols - 1 - q : q;
      const T v = tt[i] == 0 ? c[i][h] : add_in_order(c[i][h], cy[i]);
      if (e < cols && !(last_final && h == 1 && l == kWave - 1)) orow[e] = v;
    }
  }
}

// Axis 1, rows of at most NC = 16 elements (one tile each): one thread per
// row ([1000000, 8] f32 183 -> 11.6 us, [1000000, 16] 184 -> 27.8 us; 64-wide
// rows gained nothing over a wave per tile, [262144, 64] 51.4 us either
// way).  The row's real
// elements, in scan order, are positions 0 .. cols-1 of the tile's
// Hillis-Steele scan whatever the direction: forward, the
// padding zeros follow them; reversed, they precede them and every add of one
// is the same +0 as a partner below position 0.  So each step s = 1 .. 64
// adds position p - s, or +0 for p < s, exactly as the wave scan does.
constexpr int kNarrowCols = 16;
template <typename T, int NC>
__global__ __launch_bounds__(256) void cumsum_narrow_rows_kernel(const T* __restrict__ x, int64_t rows, int cols,
                                                                 int reverse, T* __restrict__ out) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const T* xr = x + r * cols;
  T* orow = out + r * cols;
  // forward rows of whole 16-byte blocks (x and out 16-byte aligned): block
  // loads and stores; otherwise one element at a time, in scan order
  const bool vec = !reverse && cols % 4 == 0 && (((uintptr_t)x | (uintptr_t)out) & 15u) == 0;
  T v[NC];
  if (vec) {
#pragma unroll
    for (int b = 0; b < NC / 4; ++b) {
      const uint4 q = b * 4 < cols ? ((const uint4*)xr)[b] : make_uint4(0u, 0u, 0u, 0u);
      v[4 * b] = __builtin_bit_cast(T, q.x);
      v[4 * b + 1] = __builtin_bit_cast(T, q.y);
      v[4 * b + 2] = __builtin_bit_cast(T, q.z);
      v[4 * b + 3] = __builtin_bit_cast(T, q.w);
    }
  } else {
#pragma unroll
    for (int p = 0; p < NC; ++p) v[p] = p < cols ? xr[reverse ? cols - 1 - p : p] : (T)0;
  }
#pragma unroll
  for (int s = 1; s < 128; s <<= 1) {
#pragma unroll
    for (int p = NC - 1; p >= 0; --p) v[p] = add_in_order(v[p], p >= s ? v[p - s] : (T)0);
  }
  if (vec) {
#pragma unroll
    for (int b = 0; b < NC / 4; ++b)
      if (b * 4 < cols)
        ((uint4*)orow)[b] = make_uint4(__builtin_bit_cast(uint32_t, v[4 * b]), __builtin_bit_cast(uint32_t, v[4 * b + 1]),
                                       __builtin_bit_cast(uint32_t, v[4 * b + 2]), __builtin_bit_cast(uint32_t, v[4 * b + 3]));
  } else {
#pragma unroll
    for (int p = 0; p < NC; ++p)
      if (p < cols) orow[reverse ? cols - 1 - p : p] = v[p];
  }
}

// Axis 0, in the same three launches: one thread per (tile of 8 rows,
// column), consecutive threads on consecutive columns.
template <typename T, bool FINAL>
__global__ __launch_bounds__(256) void cumsum_col_tiles_kernel(const T* __restrict__ x, int64_t rows, int64_t cols,
                                                               int64_t ntiles, int reverse, T* __restrict__ out) {
  const int64_t per_col = FINAL ? ntiles : ntiles - 1;
  const int64_t ntask = per_col * cols;
  const int64_t prows = ntiles * 8;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < ntask; g += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = g / cols, c = g - t * cols;
    T v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t q = t * 8 + i;
      const int64_t rr = reverse ? prows - 1 - q : q;
      v[i] = rr < rows ? x[rr * cols + c] : (T)0;
    }
    const T cy = (FINAL && t > 0) ? out[tile_last_pos(t - 1, 8, prows, reverse) * cols + c] : (T)0;
#pragma unroll
    for (int s = 1; s < 8; s <<= 1) {
      T n[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) n[i] = add_in_order(v[i], i >= s ? v[i - s] : (T)0);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = n[i];
    }
    if (!FINAL) {
      out[tile_stage_pos(t, 8, reverse) * cols + c] = v[7];
      continue;
    }
    const int last = t < ntiles - 1 ? 7 : 8;  // row 7 of a tile with a successor is already final
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t q = t * 8 + i;
      const int64_t rr = reverse ? prows - 1 - q : q;
      if (rr < rows && i < last) out[rr * cols + c] = t == 0 ? v[i] : add_in_order(v[i], cy);
    }
  }
}

// Sequential carries over staged tile totals: for tiles t = 1 .. ntot - 1 of
// each line, F[t] = add(total[t], F[t - 1]) (F[0] = total[0]), total[t] read
// from out[line * lstride + tile_stage_pos(t) * step] and F[t] stored at
// out[line * lstride + tile_last_pos(t) * step].  A workgroup takes `gl`
// lines (a power of two <= 64); all its threads stage a block of totals into
// LDS (16 loads in flight per thread; line_major: consecutive threads on
// consecutive tiles of a line, else on consecutive lines), lane j of wave 0
// chains line j from LDS (line-major rows, 16-byte reads and writes, 32 adds
// per stretch with no branch: one dependent add per tile), and all threads
// store the block's final values.
constexpr int kChainNT = 256;
constexpr int kChainBuf = 16384;  // LDS words (64 KiB for 4-byte T)
constexpr int kChainRun = 32;     // tiles per branch-free stretch of the chain

// add(v, chain_identity) == v bit for bit (-0.0 + -0.0 = -0.0, +0.0 + -0.0 = +0.0)
template <typename T>
__device__ __forceinline__ T chain_identity() { return (T)0; }
template <>
__device__ __forceinline__ float chain_identity<float>() { return -0.0f; }

template <typename T>
__global__ __launch_bounds__(kChainNT) void cumsum_chain_kernel(T* __restrict__ out, int64_t nlines, int64_t lstride,
                                                                int64_t step, int ts, int64_t plen, int reverse,
                                                                int64_t ntot, int gl, int line_major) {
  static_assert(sizeof(T) == 4, "4-byte totals");
  __shared__ __align__(16) T buf[kChainBuf];  // buf[line * rs + t]
  const int64_t L0 = (int64_t)blockIdx.x * gl;
  const int tb = kChainBuf / gl - kChainRun;  // tiles per block, a multiple of kChainRun
  const int rs = tb + 4;                       // LDS row stride (16-byte aligned, staggered banks)
  const int j0 = threadIdx.x;
  constexpr int kLoadBatch = 16;  // loads in flight per thread
  T acc = chain_identity<T>();
  for (int64_t t0 = 0; t0 < ntot; t0 += tb) {
    const int nb = (int)(ntot - t0 < tb ? ntot - t0 : tb);
    const int n = nb * gl;
    for (int jb = 0; jb < n; jb += kChainNT * kLoadBatch) {
      T v[kLoadBatch];
#pragma unroll
      for (int u = 0; u < kLoadBatch; ++u) {
        const int j = jb + u * kChainNT + j0;
        const int ll = line_major ? j / nb : (j & (gl - 1));
        const int ti = line_major ? j - ll * nb : j / gl;
        const int64_t line = L0 + ll;
        v[u] = (j < n && line < nlines) ? out[line * lstride + tile_stage_pos(t0 + ti, ts, reverse) * step] : (T)0;
      }
#pragma unroll
      for (int u = 0; u < kLoadBatch; ++u) {
        const int j = jb + u * kChainNT + j0;
        const int ll = line_major ? j / nb : (j & (gl - 1));
        const int ti = line_major ? j - ll * nb : j / gl;
        if (j < n) buf[ll * rs + ti] = v[u];
      }
    }
    __syncthreads();
    if (j0 < gl) {
      // stretches past nb read and rewrite LDS words that are never stored
      // to memory; acc is then spent (only the last block is partial)
      uint4* row = (uint4*)(buf + j0 * rs);
      for (int i0 = 0; i0 < nb; i0 += kChainRun) {
        uint4 q[kChainRun / 4];
#pragma unroll
        for (int u = 0; u < kChainRun / 4; ++u) q[u] = row[i0 / 4 + u];
#pragma unroll
        for (int u = 0; u < kChainRun / 4; ++u) {
          acc = add_in_order(__builtin_bit_cast(T, q[u].x), acc);
          q[u].x = __builtin_bit_cast(uint32_t, acc);
          acc = add_in_order(__builtin_bit_cast(T, q[u].y), acc);
          q[u].y = __builtin_bit_cast(uint32_t, acc);
          acc = add_in_order(__builtin_bit_cast(T, q[u].z), acc);
          q[u].z = __builtin_bit_cast(uint32_t, acc);
          acc = add_in_order(__builtin_bit_cast(T, q[u].w), acc);
          q[u].w = __builtin_bit_cast(uint32_t, acc);
        }
#pragma unroll
        for (int u = 0; u < kChainRun / 4; ++u) row[i0 / 4 + u] = q[u];
      }
    }
    __syncthreads();
    for (int j = j0; j < n; j += kChainNT) {
      const int ll = line_major ? j / nb : (j & (gl - 1));
      const int ti = line_major ? j - ll * nb : j / gl;
      const int64_t line = L0 + ll;
      if (line < nlines) out[line * lstride + tile_last_pos(t0 + ti, ts, plen, reverse) * step] = buf[ll * rs + ti];
    }
    __syncthreads();
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


// One workgroup per row pays off for >= 256 rows of >= 64 tiles (measured on
// f32: [256, 128256] 84 us against 114 us in three launches, [512, 32768]
// 46 against 63, [2048, 8192] 50 against 62); fewer rows leave CUs idle and
// shorter rows leave its waves idle ([4096, 4096] 83 against 63 us,
// [1024, 2048] 21.3 against 18.8), so those take the three launches.
constexpr int64_t kRowKernelMinRows = 256;
constexpr int64_t kRowKernelMinTiles = 64;

// cumsum as tile totals -> sequential chain over them -> rescan plus carry
// (one launch when every line is a single tile).
template <typename T>
static void cumsum_three_launch(const T* x, int64_t rows, int64_t cols, int axis, int reverse, T* out,
                                hipStream_t stream) {
  const int ts = axis == 1 ? 128 : 8;
  const int64_t len = axis == 1 ? cols : rows;
  const int64_t nlines = axis == 1 ? rows : cols;
  const int64_t ntiles = (len + ts - 1) / ts;
  auto tile_grid = [&](int64_t per_line) -> unsigned {
    const int64_t tasks = per_line * nlines;
    const int64_t per_block = axis == 1 ? (int64_t)kTileWaves * kTilesPerWave : 256;
    const int64_t b = (tasks + per_block - 1) / per_block;
    return (unsigned)(b > 2147483647 ? 2147483647 : b);
  };
  const unsigned tile_nt = axis == 1 ? kTileWaves * kWave : 256;
  if (ntiles > 1) {
    if (axis == 1)
      hipLaunchKernelGGL((cumsum_row_tiles_kernel<T, false>), dim3(tile_grid(ntiles - 1)), dim3(tile_nt), 0, stream,
                         x, rows, cols, ntiles, reverse, out);
    else
      hipLaunchKernelGGL((cumsum_col_tiles_kernel<T, false>), dim3(tile_grid(ntiles - 1)), dim3(tile_nt), 0, stream,
                         x, rows, cols, ntiles, reverse, out);
    // lines per chain workgroup: enough workgroups to spread the loads, the
    // lanes of wave 0 chaining their lines side by side
    int gl = 1;
    while (gl < 64 && nlines / (gl * 2) >= 256) gl *= 2;
    const int64_t cgrid = (nlines + gl - 1) / gl;
    hipLaunchKernelGGL(cumsum_chain_kernel<T>, dim3((unsigned)cgrid), dim3(kChainNT), 0, stream, out, nlines,
                       axis == 1 ? cols : (int64_t)1, axis == 1 ? (int64_t)1 : cols, ts, ntiles * ts, reverse,
                       ntiles - 1, gl, axis == 1 ? 1 : 0);
  }
  if (axis == 1)
    hipLaunchKernelGGL((cumsum_row_tiles_kernel<T, true>), dim3(tile_grid(ntiles)), dim3(tile_nt), 0, stream, x,
                       rows, cols, ntiles, reverse, out);
  else
    hipLaunchKernelGGL((cumsum_col_tiles_kernel<T, true>), dim3(tile_grid(ntiles)), dim3(tile_nt), 0, stream, x,
                       rows, cols, ntiles, reverse, out);
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
    const int64_t lds_max = irows >= kGatherManyRows ? kGatherLdsMaxMany : kGatherLdsMax;
    if (vcols * es <= lds_max && irows <= 2147483647) {
      const size_t lds = (size_t)vcols * es;
      const void* kern = es == 2 ? (const void*)gather_row_lds_kernel<uint16_t> : (const void*)gather_row_lds_kernel<uint32_t>;
      if (lds > 64 * 1024) {
        const hipError_t attr = set_dynamic_lds_limit(kern, (int)lds, stream);
        if (attr != hipSuccess) {
          set_error("hipFuncSetAttribute: %s", hipGetErrorString(attr));
          return kHipError;
        }
      }
      if (es == 2)
        hipLaunchKernelGGL(gather_row_lds_kernel<uint16_t>, dim3((unsigned)irows), dim3(kGatherNT), lds, stream,
                           (const uint16_t*)values, vcols, indices, icols, (uint16_t*)out);
      else
        hipLaunchKernelGGL(gather_row_lds_kernel<uint32_t>, dim3((unsigned)irows), dim3(kGatherNT), lds, stream,
                           (const uint32_t*)values, vcols, indices, icols, (uint32_t*)out);
    } else if (irows * 64 <= 2147483647 / 8 && icols >= 64 * 256) {
      // chunks of >= 256 outputs, ~64 per row
      const int64_t chunks = 64;
      const unsigned grid = (unsigned)(8 * ((irows + 7) / 8) * chunks);
      if (es == 2)
        hipLaunchKernelGGL(gather_row_xcd_kernel<uint16_t>, dim3(grid), dim3(256), 0, stream, (const uint16_t*)values,
                           vcols, indices, icols, irows, chunks, (uint16_t*)out);
      else
        hipLaunchKernelGGL(gather_row_xcd_kernel<uint32_t>, dim3(grid), dim3(256), 0, stream, (const uint32_t*)values,
                           vcols, indices, icols, irows, chunks, (uint32_t*)out);
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
  {
    const uintptr_t xb = (uintptr_t)x, ob = (uintptr_t)out, nb = (uintptr_t)(rows * cols) * 4u;
    if (xb < ob + nb && ob < xb + nb) {
      set_error("cumsum out must not overlap x (tile totals are staged in out)");
      return kInvalidArgument;
    }
  }
  if (axis == 1 && cols <= kNarrowCols) {
    const unsigned grid = (unsigned)((rows + 255) / 256);
    if (dtype == kF32)
      hipLaunchKernelGGL((cumsum_narrow_rows_kernel<float, kNarrowCols>), dim3(grid), dim3(256), 0, stream,
                         (const float*)x, rows, (int)cols, reverse, (float*)out);
    else
      hipLaunchKernelGGL((cumsum_narrow_rows_kernel<int32_t, kNarrowCols>), dim3(grid), dim3(256), 0, stream,
                         (const int32_t*)x, rows, (int)cols, reverse, (int32_t*)out);
  } else if (axis == 1) {
    const int64_t ntiles = (cols + 127) / 128;
    if (rows >= kRowKernelMinRows && ntiles >= kRowKernelMinTiles && rows <= 2147483647) {
      if (dtype == kF32)
        hipLaunchKernelGGL(cumsum_rows_kernel<float>, dim3((unsigned)rows), dim3(kScanNT), 0, stream,
                           (const float*)x, cols, reverse, (float*)out);
      else
        hipLaunchKernelGGL(cumsum_rows_kernel<int32_t>, dim3((unsigned)rows), dim3(kScanNT), 0, stream,
                           (const int32_t*)x, cols, reverse, (int32_t*)out);
    } else if (dtype == kF32) {
      cumsum_three_launch<float>((const float*)x, rows, cols, 1, reverse, (float*)out, stream);
    } else {
      cumsum_three_launch<int32_t>((const int32_t*)x, rows, cols, 1, reverse, (int32_t*)out, stream);
    }
  } else if (dtype == kF32) {
    cumsum_three_launch<float>((const float*)x, rows, cols, 0, reverse, (float*)out, stream);
  } else {
    cumsum_three_launch<int32_t>((const int32_t*)x, rows, cols, 0, reverse, (int32_t*)out, stream);
  }
  return launch_status("tallax_cumsum");
}

}  // extern "C"
