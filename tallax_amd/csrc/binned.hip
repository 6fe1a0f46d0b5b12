// Approximate (binned) top-k for gfx950: tax.top_dynamic_k with
// guarantee_convergence=False.
//
// Reference semantics (tallax/_src/top_k.py:13-106, 203-370, 372-514):
//   * bin b holds the columns j = b (mod num_bins); each bin keeps its m
//     largest values in index order with a strict-> sinking insert, so ties
//     keep the lower index and values <= finfo.min or NaN never enter;
//   * for each schedule step m: pivot = max over bins of the m-th largest,
//     num_larger = #(entries of ranks < m-1 that are >= pivot); a row
//     converges when num_larger >= k[row] (depth = m-1 at the first
//     convergence, max_k otherwise); steps are evaluated for a block of
//     block_token rows until every row of the block converged; cutoff = the
//     pivot of the last evaluated step;
//   * valid = (max depth over all rows < schedule[-1]) or schedule[-1] == max_k;
//   * the result is the top-128 of the first depth_upper ranks of every bin
//     (depth_upper = the power-of-two bucket of the global max depth),
//     truncated to max_k, with replace_val at positions >= k[row].
// The ranks inside a bin are the same whatever the pass structure (each pass
// extends the exact per-bin top-m), so one scan computes the deepest lists
// and every step's statistics.
//
// Kernels:
//   binned_lists_kernel  one workgroup per row: thread (bin, slice) scans
//                        every S-th element of its bin keeping a register
//                        top-MC list; the slices of a bin are merged through
//                        LDS; ranks < buf go to the workspace with each
//                        step's (pivot, count).
//   binned_finish_kernel one workgroup: depths, cutoffs, valid, depth_upper.
//   binned_select_kernel one workgroup per row: bitonic sort of the
//                        depth_upper * num_bins superset, top-128 out.
#include <float.h>
#include <stdint.h>
#include <string.h>

#include "tallax_hip.h"
#include "tx_common.h"
#include "tx_host.h"
#include "tx_wave_sort.h"

namespace tx {

constexpr int kBinNT = 1024;
constexpr int kMaxSteps = 16;

struct BinArgs {
  const void* x;
  int dtype;
  int64_t rows, cols;
  const int32_t* k_rows;
  int max_k;
  int block_token;
  int num_bins;
  int buf;                 // ranks kept per bin
  int nsteps;              // schedule steps (leading 0 excluded)
  int steps[kMaxSteps];
  int gsched[kMaxSteps + 1];  // power-of-two depth buckets, ascending
  int ngs;
  int has_replace;
  float replace_val;       // in the input dtype
  void* out_vals;
  int32_t* out_idx;
  int32_t* out_valid;
  int32_t* out_depths;
  float* out_cutoff;
  // workspace
  float* lv;               // [rows][buf][num_bins]
  int32_t* li;             // [rows][buf][num_bins]
  float* st_pivot;         // [rows][nsteps]
  int32_t* st_count;       // [rows][nsteps]
  int32_t* upper;          // [1]
};

__device__ __forceinline__ float load_val(const void* x, int dt, int64_t i) {
  return dt == kBF16 ? __uint_as_float(((uint32_t)((const uint16_t*)x)[i]) << 16) : ((const float*)x)[i];
}
__device__ __forceinline__ float dtype_min_f(int dt) {
  return dt == kBF16 ? __uint_as_float(0xFF7F0000u) : -FLT_MAX;
}
// (value desc, index asc) order: a before b
__device__ __forceinline__ bool ahead(float va, int32_t ia, float vb, int32_t ib) {
  return va > vb || (va == vb && (uint32_t)ia < (uint32_t)ib);
}

template <int MC>
__global__ __launch_bounds__(kBinNT) void binned_lists_kernel(BinArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int NB = a.num_bins;
  const int S = kBinNT / NB;  // slices per bin
  float* sv = (float*)smem;                         // [S][MC][NB]
  int32_t* si = (int32_t*)(sv + (size_t)S * MC * NB);
  __shared__ float red_f[kBinNT / kWave];
  __shared__ int red_i[kBinNT / kWave];
  const int t = threadIdx.x;
  const int b = t % NB, s = t / NB;
  const int64_t row = blockIdx.x;
  const float lo = dtype_min_f(a.dtype);
  float v[MC];
  int32_t id[MC];
#pragma unroll
  for (int r = 0; r < MC; ++r) {
    v[r] = lo;
    id[r] = -1;
  }
  // slice s of bin b: columns b + NB * (s + S * i), in index order
  const int64_t base = row * a.cols;
  const int step = NB * S;  // = kBinNT
  // 16 loads in flight per thread (one workgroup per row: each CU needs deep
  // memory-level parallelism), then the inserts in index order
  constexpr int U = MC <= 8 ? 16 : 8;
  const int j0 = s * NB + b;
  for (int64_t jb = j0; jb < a.cols; jb += (int64_t)U * step) {
    float xs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = jb + (int64_t)u * step;
      xs[u] = j < a.cols ? load_val(a.x, a.dtype, base + j) : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float x = xs[u];
      if (x > v[MC - 1]) {  // strict: ties keep the earlier (lower) index; NaN never enters
        int32_t xi = (int32_t)(jb + (int64_t)u * step);
#pragma unroll
        for (int r = 0; r < MC; ++r) {
          const bool sw = x > v[r];
          const float tv = v[r];
          const int32_t ti = id[r];
          v[r] = sw ? x : tv;
          id[r] = sw ? xi : ti;
          x = sw ? tv : x;
          xi = sw ? ti : xi;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < MC; ++r) {
    sv[((size_t)s * MC + r) * NB + b] = v[r];
    si[((size_t)s * MC + r) * NB + b] = id[r];
  }
  // fillers for every rank of this bin's output list (real entries overwrite them)
  for (int r = s; r < a.buf; r += S) {
    a.lv[((size_t)row * a.buf + r) * NB + b] = lo;
    a.li[((size_t)row * a.buf + r) * NB + b] = -1;
  }
  __syncthreads();
  // merged rank of each own entry among the bin's S x MC pool (value desc,
  // index asc); real entries only
  int rank[MC];
  int nreal = 0;  // real entries in the bin
#pragma unroll
  for (int r = 0; r < MC; ++r) rank[r] = 0;
  for (int q = 0; q < S; ++q) {
    for (int h = 0; h < MC; ++h) {
      const int32_t ci = si[((size_t)q * MC + h) * NB + b];
      if (ci < 0) continue;
      const float cv = sv[((size_t)q * MC + h) * NB + b];
      ++nreal;
#pragma unroll
      for (int r = 0; r < MC; ++r) rank[r] += ahead(cv, ci, v[r], id[r]) ? 1 : 0;
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < MC; ++r) {
    if (id[r] >= 0 && rank[r] < a.buf) {
      a.lv[((size_t)row * a.buf + rank[r]) * NB + b] = v[r];
      a.li[((size_t)row * a.buf + rank[r]) * NB + b] = id[r];
    }
  }
  // statistics of every schedule step from the ranked entries
  const int w = t / kWave, l = lane_id();
  constexpr int NW = kBinNT / kWave;
  const int kept = nreal < MC ? nreal : MC;  // real entries in the bin's merged list
  for (int q = 0; q < a.nsteps; ++q) {
    const int m = a.steps[q];
    float pv = -INFINITY;
#pragma unroll
    for (int r = 0; r < MC; ++r)
      if (id[r] >= 0 && rank[r] == m - 1) pv = fmaxf(pv, v[r]);
    if (s == 0 && kept < m) pv = fmaxf(pv, lo);  // the bin's m-th entry is a filler
#pragma unroll
    for (int d = kWave / 2; d >= 1; d >>= 1) pv = fmaxf(pv, lane_xor_f(pv, d));
    if (l == 0) red_f[w] = pv;
    __syncthreads();
    float pivot = red_f[0];
    for (int i = 1; i < NW; ++i) pivot = fmaxf(pivot, red_f[i]);
    int c = 0;
#pragma unroll
    for (int r = 0; r < MC; ++r) c += (id[r] >= 0 && rank[r] < m - 1 && v[r] >= pivot) ? 1 : 0;
    if (s == 0 && lo >= pivot) c += (m - 1) - (kept < m - 1 ? kept : m - 1);  // fillers above the pivot
    c = wave_sum_i(c);
    if (l == 0) red_i[w] = c;
    __syncthreads();
    if (t == 0) {
      int tot = 0;
      for (int i = 0; i < NW; ++i) tot += red_i[i];
      a.st_pivot[row * a.nsteps + q] = pivot;
      a.st_count[row * a.nsteps + q] = tot;
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void binned_finish_kernel(BinArgs a) {
  __shared__ int red[256 / kWave];
  const int t = threadIdx.x;
  const int64_t nblk = a.rows / a.block_token;
  int gmax = 0;
  for (int64_t bk = t; bk < nblk; bk += blockDim.x) {
    const int64_t r0 = bk * a.block_token;
    for (int i = 0; i < a.block_token; ++i) a.out_depths[r0 + i] = a.max_k;
    for (int q = 0; q < a.nsteps; ++q) {
      const int m = a.steps[q];
      bool all = true;
      for (int i = 0; i < a.block_token; ++i) {
        const int64_t r = r0 + i;
        const bool conv = a.st_count[r * a.nsteps + q] >= a.k_rows[r];
        if (conv && a.out_depths[r] == a.max_k) a.out_depths[r] = m - 1;
        a.out_cutoff[r] = a.st_pivot[r * a.nsteps + q];
        all = all && conv;
      }
      if (all) break;
    }
    for (int i = 0; i < a.block_token; ++i) gmax = max(gmax, a.out_depths[r0 + i]);
  }
  const int l = lane_id();
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) gmax = max(gmax, (int)lane_xor((uint32_t)gmax, d));
  if (l == 0) red[t / kWave] = gmax;
  __syncthreads();
  if (t == 0) {
    int g = 0;
    for (int i = 0; i < (int)(blockDim.x / kWave); ++i) g = max(g, red[i]);
    a.out_valid[0] = (g < a.steps[a.nsteps - 1] || a.steps[a.nsteps - 1] == a.max_k) ? 1 : 0;
    int up = a.gsched[a.ngs - 1];
    for (int i = 0; i + 1 < a.ngs; ++i) {
      if (a.gsched[i] < g && g <= a.gsched[i + 1]) {
        up = a.gsched[i + 1];
        break;
      }
    }
    a.upper[0] = up;
  }
}

// composite of a list entry: value descending then index ascending; fillers
// (index -1) after every real entry
__device__ __forceinline__ uint64_t entry_comp(float v, int32_t i) {
  if (i < 0) return 0ull;
  return make_comp(select_key(__float_as_uint(v)), (uint32_t)i);
}

__global__ __launch_bounds__(1024) void binned_select_kernel(BinArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* lds = (uint64_t*)smem;
  const int t = threadIdx.x;
  const int NT = blockDim.x;
  const int64_t row = blockIdx.x;
  const int NB = a.num_bins;
  const int up = a.upper[0] < a.buf ? a.upper[0] : a.buf;
  const int n = up * NB;
  int P = 1;
  while (P < n) P <<= 1;
  for (int i = t; i < P; i += NT) {
    uint64_t c = 0;
    if (i < n) {
      const int r = i / NB, b = i % NB;
      c = entry_comp(a.lv[((size_t)row * a.buf + r) * NB + b], a.li[((size_t)row * a.buf + r) * NB + b]);
    }
    lds[i] = c;
  }
  __syncthreads();
  // bitonic sort, descending
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride >= 1; stride >>= 1) {
      for (int i = t; i < P; i += NT) {
        const int j = i ^ stride;
        if (j > i) {
          const uint64_t x = lds[i], y = lds[j];
          const bool desc = (i & size) == 0;
          if ((x < y) == desc) {
            lds[i] = y;
            lds[j] = x;
          }
        }
      }
      __syncthreads();
    }
  }
  const float lo = dtype_min_f(a.dtype);
  const int kr = a.k_rows[row];
  for (int p = t; p < a.max_k; p += NT) {
    const uint64_t c = p < P ? lds[p] : 0ull;
    float v = lo;
    int32_t id = -1;
    if (c != 0ull) {
      v = __uint_as_float(key_to_bits(comp_key(c)));
      id = comp_idx(c);
    }
    if (a.has_replace && p >= kr) v = a.replace_val;
    const int64_t o = row * a.max_k + p;
    if (a.dtype == kBF16)
      ((uint16_t*)a.out_vals)[o] = (uint16_t)(__float_as_uint(v) >> 16);
    else
      ((float*)a.out_vals)[o] = v;
    a.out_idx[o] = id;
  }
}

static int log2_ceil(int x) {
  int r = 0;
  while ((1 << r) < x) ++r;
  return r;
}

static int bin_buf(int max_m) { return max_m > 1 ? (max_m > (1 << log2_ceil(max_m - 1)) ? max_m : (1 << log2_ceil(max_m - 1))) : max_m; }

static size_t bin_ws(int64_t rows, int num_bins, int buf, int nsteps) {
  size_t b = 0;
  b += (size_t)rows * buf * num_bins * 4;  // lv
  b += (size_t)rows * buf * num_bins * 4;  // li
  b += (size_t)rows * nsteps * 4;          // pivots
  b += (size_t)rows * nsteps * 4;          // counts
  b += 256;
  return align_up(b, 256);
}

}  // namespace tx

using namespace tx;

extern "C" {

size_t tallax_top_dynamic_k_workspace_size(int64_t rows, int num_bins, const int32_t* schedule, int num_steps) {
  if (rows < 0 || num_bins <= 0 || !schedule || num_steps <= 0 || num_steps > kMaxSteps) return 0;
  return bin_ws(rows, num_bins, bin_buf(schedule[num_steps - 1]), num_steps);
}

int tallax_top_dynamic_k(const void* x, int dtype, int64_t rows, int64_t cols, const int32_t* k_rows, int max_k,
                         int block_token, int num_bins, const int32_t* schedule, int num_steps, int has_replace,
                         double replace_val, void* out_vals, int32_t* out_idx, int32_t* out_valid,
                         int32_t* out_depths, float* out_cutoff, void* workspace, size_t workspace_bytes,
                         hipStream_t stream) {
  if (!x || !k_rows || !schedule || !out_vals || !out_idx || !out_valid || !out_depths || !out_cutoff) {
    set_error("null pointer argument");
    return kInvalidArgument;
  }
  if (dtype != kF32 && dtype != kBF16) { set_error("dtype %d not supported (f32=0, bf16=1)", dtype); return kUnsupported; }
  if (rows < 0 || cols <= 0) { set_error("bad shape [%lld, %lld]", (long long)rows, (long long)cols); return kInvalidArgument; }
  if (max_k < 1 || max_k > 128) { set_error("max_k=%d outside [1, 128]", max_k); return max_k > 128 ? kUnsupported : kInvalidArgument; }
  if (block_token < 1 || rows % block_token) { set_error("num_tokens must be divisible by block_token"); return kInvalidArgument; }
  if (num_bins < 1 || num_bins > kBinNT || (kBinNT % num_bins)) {
    set_error("num_bins=%d must divide %d", num_bins, kBinNT);
    return kUnsupported;
  }
  if (num_steps < 1 || num_steps > kMaxSteps) { set_error("schedule of %d steps unsupported", num_steps); return kUnsupported; }
  for (int q = 0; q < num_steps; ++q) {
    if (schedule[q] < 1 || (q && schedule[q] <= schedule[q - 1])) {
      set_error("schedule must be strictly increasing positive depths");
      return kInvalidArgument;
    }
  }
  if (cols >= (int64_t)1 << 31) { set_error("cols must fit int32 indices"); return kInvalidArgument; }
  if (rows == 0) return kOk;
  const int max_m = schedule[num_steps - 1];
  const int buf = bin_buf(max_m);
  if (buf > 16) { set_error("schedule depth %d exceeds this build's per-bin list of 16", max_m); return kUnsupported; }
  const size_t need = bin_ws(rows, num_bins, buf, num_steps);
  if (!workspace || workspace_bytes < need) {
    set_error("workspace of %zu bytes is smaller than the %zu required", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  BinArgs a = {};
  a.x = x; a.dtype = dtype; a.rows = rows; a.cols = cols; a.k_rows = k_rows; a.max_k = max_k;
  a.block_token = block_token; a.num_bins = num_bins; a.buf = buf; a.nsteps = num_steps;
  for (int q = 0; q < num_steps; ++q) a.steps[q] = schedule[q];
  // power-of-two buckets of (0, schedule...): 2^ceil(log2(m - 1)) for m > 1
  int gs[kMaxSteps + 1];
  int ng = 0;
  auto add = [&](int v) {
    for (int i = 0; i < ng; ++i) if (gs[i] == v) return;
    gs[ng++] = v;
  };
  add(0);
  for (int q = 0; q < num_steps; ++q) add(schedule[q] > 1 ? (1 << log2_ceil(schedule[q] - 1)) : schedule[q]);
  for (int i = 0; i < ng; ++i)
    for (int j = i + 1; j < ng; ++j)
      if (gs[j] < gs[i]) { const int tmp = gs[i]; gs[i] = gs[j]; gs[j] = tmp; }
  for (int i = 0; i < ng; ++i) a.gsched[i] = gs[i];
  a.ngs = ng;
  a.has_replace = has_replace != 0;
  float rv = (float)replace_val;
  if (dtype == kBF16) {  // round to bfloat16, nearest even
    uint32_t u;
    memcpy(&u, &rv, 4);
    u = ((u & 0x7fffffffu) > 0x7f800000u) ? ((u | 0x00400000u) & 0xffff0000u) : ((u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u);
    memcpy(&rv, &u, 4);
  }
  a.replace_val = rv;
  a.out_vals = out_vals; a.out_idx = out_idx; a.out_valid = out_valid; a.out_depths = out_depths;
  a.out_cutoff = out_cutoff;
  char* w = (char*)workspace;
  a.lv = (float*)w;
  w += (size_t)rows * buf * num_bins * 4;
  a.li = (int32_t*)w;
  w += (size_t)rows * buf * num_bins * 4;
  a.st_pivot = (float*)w;
  w += (size_t)rows * num_steps * 4;
  a.st_count = (int32_t*)w;
  w += (size_t)rows * num_steps * 4;
  a.upper = (int32_t*)w;
  if (rows > 2147483647) { set_error("too many rows"); return kUnsupported; }
  // kernel 1
  const int S = kBinNT / num_bins;
  const int mc = buf <= 8 ? 8 : 16;
  const size_t lds = (size_t)S * mc * num_bins * 8;  // = kBinNT * mc * 8 <= 128 KiB
  static const hipError_t attr8 = hipFuncSetAttribute((const void*)binned_lists_kernel<8>,
                                                      hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024);
  static const hipError_t attr16 = hipFuncSetAttribute((const void*)binned_lists_kernel<16>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024);
  if (attr8 != hipSuccess || attr16 != hipSuccess) {
    set_error("hipFuncSetAttribute failed");
    return kHipError;
  }
  if (mc == 8)
    hipLaunchKernelGGL(binned_lists_kernel<8>, dim3((unsigned)rows), dim3(kBinNT), lds, stream, a);
  else
    hipLaunchKernelGGL(binned_lists_kernel<16>, dim3((unsigned)rows), dim3(kBinNT), lds, stream, a);
  int st = launch_status("tallax_top_dynamic_k");
  if (st) return st;
  hipLaunchKernelGGL(binned_finish_kernel, dim3(1), dim3(256), 0, stream, a);
  st = launch_status("tallax_top_dynamic_k");
  if (st) return st;
  // kernel 3: the superset is at most gsched[last] * num_bins entries
  const int max_up = a.gsched[a.ngs - 1] < buf ? a.gsched[a.ngs - 1] : buf;
  int P = 1;
  while (P < max_up * num_bins) P <<= 1;
  const size_t lds3 = (size_t)P * 8;
  if (lds3 > 160 * 1024) { set_error("superset of %d entries does not fit LDS", P); return kUnsupported; }
  static const hipError_t attr3 = hipFuncSetAttribute((const void*)binned_select_kernel,
                                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  if (attr3 != hipSuccess) { set_error("hipFuncSetAttribute failed"); return kHipError; }
  hipLaunchKernelGGL(binned_select_kernel, dim3((unsigned)rows), dim3(1024), lds3, stream, a);
  return launch_status("tallax_top_dynamic_k");
}

}  // extern "C"
