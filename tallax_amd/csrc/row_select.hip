// Exact row top-k (k <= 128) and the fused top-k / top-p / temperature /
// Gumbel-max sampler for gfx950.
//
// Reference semantics:
//   * tax.top_k = top_dynamic_k(..., guarantee_convergence=True)
//     (tallax/_src/top_k.py:516-567): values descending, ties broken to the
//     lowest index; NaN, -inf and finfo.min are never selected (the bins start
//     at finfo.min and admit only strictly greater values, top_k.py:64,241).
//   * sampling.sample (tallax/_src/sampling.py:331-343): top-128 with positions
//     >= top_k[row] replaced by replace_val in the logits dtype (top_k.py:365-369,
//     sampling.py:283-290), then top_p_and_sample_arrays (sampling.py:65-115).
//
// Design (each element is read from HBM exactly once):
//   Kernel A, seg_select_kernel: a row is cut into `nseg` segments, one
//   256-thread workgroup each, sized so that ~4 workgroups run per CU.  A
//   workgroup streams its segment in tiles of 256 x V 16-byte vectors held in
//   registers, prefetching tile t+1 while it filters tile t:
//     - every element becomes a monotone 32-bit select key;
//     - tile 0 sets a lower bound L on the segment's k-th key: each wave sorts
//       its 64 per-thread maxima (wave64 bitonic network) and L is the minimum
//       over the 4 waves of their ceil(k/4)-th largest maximum, so at least k
//       elements are >= L;
//     - elements passing the current filter become candidates (u64 composite
//       key << 32 | ~index) in an LDS buffer; once it holds more than 512 the
//       buffer is cut to its exact top-k and the filter tightens to
//       "key > key of the k-th" (later elements have larger indices, so an
//       equal key can no longer win a tie);
//     - a tile with more than 512 candidates (heavy ties) contributes its
//       exact top-k instead, found by bisection on the composite key.
//   Selection sorts 128-element runs with a wave64 bitonic network and merges
//   runs with bitonic merge-and-discard (tx_wave_sort.h).
//   Kernel B, seg_merge_kernel (only when nseg > 1): one wave per row merges
//   the segment lists and writes (values, indices) or runs the sampler tail.
//   The kernel boundary orders the workspace writes before the reads, so no
//   device-scope fence (an L2 write-back on gfx950) is ever issued.
#include <float.h>
#include <math.h>
#include <string.h>

#include "tallax_hip.h"
#include "tx_common.h"
#include "tx_host.h"
#include "tx_math.h"
#include "tx_sample.h"
#include "tx_wave_sort.h"

namespace tx {

constexpr int kNT = 256;                   // threads per workgroup: 4 wave64s
constexpr int kWaves = kNT / kWave;
constexpr int kCap = 1024;                 // LDS candidate slots
constexpr int kTileCap = 512;              // candidates one tile may add directly
constexpr int kRefresh = kCap - kTileCap;  // cut the buffer to top-k above this
constexpr int kMaxK = 128;                 // the reference's limit (top_k.py:438-439)
constexpr int kRun = 128;                  // list length handed between kernels
constexpr int kMaxSeg = 16;
constexpr int kTargetBlocks = 1024;        // ~4 workgroups per CU on 256 CUs
constexpr int kVF32 = 8;                   // 16-byte vectors per thread per tile
constexpr int kVBF16 = 4;

struct SelArgs {
  const void* x;
  int64_t rows, cols;
  int k;
  int nseg;
  int64_t vps;  // 16-byte vectors per segment
  // top-k outputs
  void* out_vals;
  int32_t* out_idx;
  // segment lists: rows * nseg * kRun composites
  uint64_t* ws_lists;
  // sampler
  const int32_t* top_k;
  const float* top_p;
  const float* temperature;
  const uint32_t* rng_key;
  int64_t dim0_offset;
  float replace_in_dtype;  // replace_val rounded to the logits dtype
  float replace_f32;       // replace_val rounded to float32
  int32_t* out_tokens;
};

template <int DT>
struct ElemT;
template <>
struct ElemT<kF32> {
  static constexpr int VEC = 4, ES = 4;
  __device__ static __forceinline__ uint32_t bits(const uint4& v, int q) {
    return q == 0 ? v.x : q == 1 ? v.y : q == 2 ? v.z : v.w;
  }
  __device__ static __forceinline__ uint32_t load_bits(const void* row, int64_t i) {
    return ((const uint32_t*)row)[i];
  }
  __device__ static __forceinline__ void store(void* out, int64_t i, uint32_t b) {
    ((uint32_t*)out)[i] = b;
  }
  static constexpr uint32_t kMinBits = 0xff7fffffu;  // finfo(float32).min
};
template <>
struct ElemT<kBF16> {
  static constexpr int VEC = 8, ES = 2;
  __device__ static __forceinline__ uint32_t bits(const uint4& v, int q) {
    const int w = q >> 1;
    const uint32_t x = w == 0 ? v.x : w == 1 ? v.y : w == 2 ? v.z : v.w;
    return (q & 1) ? (x & 0xffff0000u) : (x << 16);
  }
  __device__ static __forceinline__ uint32_t load_bits(const void* row, int64_t i) {
    return ((uint32_t)((const uint16_t*)row)[i]) << 16;
  }
  __device__ static __forceinline__ void store(void* out, int64_t i, uint32_t b) {
    ((uint16_t*)out)[i] = (uint16_t)(b >> 16);
  }
  static constexpr uint32_t kMinBits = 0xff7f0000u;  // finfo(bfloat16).min, widened
};

struct SegShared {
  uint64_t cand[kCap];
  uint64_t scratch[kWaves * kRun];
  uint64_t list[kRun];
  uint32_t wl[kWaves];
  int red[kWaves];
  int cnt;
};

__device__ __forceinline__ int block_sum(int v, int* red) {
  v = wave_sum_i(v);
  __syncthreads();
  if (lane_id() == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) t += red[i];
  return t;
}

// sh.list <- the 128 largest of sh.cand[0, C), descending, zero padded.
__device__ void block_select(SegShared& sh, int C) {
  const int w = threadIdx.x / kWave, l = lane_id();
  uint64_t acc[2] = {0, 0};
  bool any = false;
  for (int r = w; r * kRun < C; r += kWaves) {
    uint64_t c[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = r * kRun + h * kWave + l;
      c[h] = i < C ? sh.cand[i] : 0ull;
    }
    wave_sort128_desc(c);
    if (!any) {
      acc[0] = c[0];
      acc[1] = c[1];
      any = true;
    } else {
      wave_merge128_desc(acc, c);
    }
  }
  sh.scratch[w * kRun + l] = acc[0];
  sh.scratch[w * kRun + kWave + l] = acc[1];
  __syncthreads();
  if (w == 0) {
    const int runs = (C + kRun - 1) / kRun;
    const int nw = runs < kWaves ? runs : kWaves;
    for (int q = 1; q < nw; ++q) {
      const uint64_t b[2] = {sh.scratch[q * kRun + l], sh.scratch[q * kRun + kWave + l]};
      wave_merge128_desc(acc, b);
    }
    sh.list[l] = acc[0];
    sh.list[kWave + l] = acc[1];
  }
  __syncthreads();
}

// Outputs of one row from its sorted top-128 list (in LDS).
template <int DT, bool SAMPLE>
__device__ void finalize_row(const SelArgs& a, int64_t row, const uint64_t* list) {
  using T = ElemT<DT>;
  const uint32_t inel = ineligible_key_max(DT);
  const char* rowp = (const char*)a.x + (size_t)(row * a.cols) * T::ES;
  if (!SAMPLE) {
    for (int i = threadIdx.x; i < a.k; i += blockDim.x) {
      const uint64_t c = list[i];
      const uint32_t kk = comp_key(c);
      const int32_t idx = comp_idx(c);
      const uint32_t b = kk > inel ? T::load_bits(rowp, idx) : T::kMinBits;
      T::store(a.out_vals, row * a.k + i, b);
      a.out_idx[row * a.k + i] = idx;
    }
  } else if (threadIdx.x < kWave) {
    const int l = lane_id();
    const int kr = a.top_k[row];
    float v[2];
    int32_t id[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int p = h * kWave + l;
      const uint64_t c = list[p];
      const uint32_t kk = comp_key(c);
      id[h] = comp_idx(c);
      const float val = __uint_as_float(kk > inel ? key_to_bits(kk) : T::kMinBits);
      v[h] = p < kr ? val : a.replace_in_dtype;
    }
    const uint32_t row_ctr = (uint32_t)(row + a.dim0_offset);
    const int32_t tok = sample_tail(v, id, kMaxK, a.top_p[row], a.temperature[row], a.rng_key[0],
                                    a.rng_key[1], row_ctr, (uint32_t)a.cols, a.replace_f32);
    if (l == 0) a.out_tokens[row] = tok;
  }
}

// ---------------------------------------------------------------------------
// Kernel A: one workgroup per (segment, row).
// ---------------------------------------------------------------------------
template <int DT, int V, bool SAMPLE>
__global__ __launch_bounds__(kNT) void seg_select_kernel(SelArgs a) {
  using T = ElemT<DT>;
  constexpr int VEC = T::VEC, ES = T::ES, E = V * VEC;
  constexpr int64_t kTileVec = (int64_t)kNT * V;
  __shared__ SegShared sh;
  const int tid = threadIdx.x;
  const int w = tid / kWave, l = lane_id();
  const int seg = blockIdx.x;
  const int64_t row = blockIdx.y;
  const int k = a.k;

  const char* rowp = (const char*)a.x + (size_t)(row * a.cols) * ES;
  const RowVec<ES> rv(rowp);
  const int64_t nv = (a.cols + rv.mis + VEC - 1) / VEC;
  const int64_t s0 = (int64_t)seg * a.vps;
  const int64_t s1 = s0 + a.vps < nv ? s0 + a.vps : nv;
  const int ntiles = s1 > s0 ? (int)((s1 - s0 + kTileVec - 1) / kTileVec) : 0;
  if (tid == 0) sh.cnt = 0;

  uint4 cur[V], nxt[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int64_t v = s0 + (int64_t)j * kNT + tid;
    cur[j] = v < s1 ? rv.base[v] : make_uint4(0u, 0u, 0u, 0u);
  }

  uint32_t thr = 1;  // candidates: key >= thr
  int base = 0;      // candidates held before the current tile
  for (int t = 0; t < ntiles; ++t) {
    const int64_t tb = s0 + (int64_t)t * kTileVec;
    if (t + 1 < ntiles) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int64_t v = tb + kTileVec + (int64_t)j * kNT + tid;
        nxt[j] = v < s1 ? rv.base[v] : make_uint4(0u, 0u, 0u, 0u);
      }
    }
    uint32_t key[E];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int64_t v = tb + (int64_t)j * kNT + tid;
      const int64_t e0 = v * VEC - rv.mis;
      const bool live = v < s1;
      const bool full = live && e0 >= 0 && e0 + VEC <= a.cols;
#pragma unroll
      for (int q = 0; q < VEC; ++q) {
        const bool ok = full || (live && e0 + q >= 0 && e0 + q < a.cols);
        key[j * VEC + q] = ok ? select_key(T::bits(cur[j], q)) : 0u;
      }
    }
    auto elem_idx = [&](int j, int q) -> uint32_t {
      return (uint32_t)((tb + (int64_t)j * kNT + tid) * VEC + q - rv.mis);
    };

    if (t == 0) {
      uint32_t tmax = 0;
#pragma unroll
      for (int i = 0; i < E; ++i) tmax = key[i] > tmax ? key[i] : tmax;
      const uint32_t srt = wave_sort64_u32_desc(tmax);
      const int jw = (k + kWaves - 1) / kWaves;
      const uint32_t wl = (uint32_t)__shfl((int)srt, jw - 1, kWave);
      if (l == 0) sh.wl[w] = wl;
      __syncthreads();
      uint32_t L = sh.wl[0];
#pragma unroll
      for (int i = 1; i < kWaves; ++i) L = sh.wl[i] < L ? sh.wl[i] : L;
      thr = L > 1u ? L : 1u;
    }

    // ---- append this tile's candidates ------------------------------------
    int c = 0;
#pragma unroll
    for (int i = 0; i < E; ++i) c += key[i] >= thr;
    int pos = c > 0 ? atomicAdd(&sh.cnt, c) : 0;
    if (c > 0 && pos + c <= kCap) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
          const uint32_t kk = key[j * VEC + q];
          if (kk >= thr) sh.cand[pos++] = make_comp(kk, elem_idx(j, q));
        }
      }
    }
    __syncthreads();
    int total = sh.cnt;
    __syncthreads();

    if (total - base > kTileCap) {
      // Heavy ties: keep only this tile's exact top-k among the passing
      // elements (composites are distinct, so exactly k pass the bisection).
      uint64_t prefix = 0;
      for (int bit = 63; bit >= 0; --bit) {
        const uint64_t probe = prefix | (1ull << bit);
        int cc = 0;
#pragma unroll
        for (int j = 0; j < V; ++j) {
#pragma unroll
          for (int q = 0; q < VEC; ++q) {
            const uint32_t kk = key[j * VEC + q];
            cc += kk >= thr && make_comp(kk, elem_idx(j, q)) >= probe;
          }
        }
        if (block_sum(cc, sh.red) >= k) prefix = probe;
      }
      if (tid == 0) sh.cnt = base;
      __syncthreads();
      int cc = 0;
#pragma unroll
      for (int j = 0; j < V; ++j) {
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
          const uint32_t kk = key[j * VEC + q];
          cc += kk >= thr && make_comp(kk, elem_idx(j, q)) >= prefix;
        }
      }
      int p2 = cc > 0 ? atomicAdd(&sh.cnt, cc) : 0;
#pragma unroll
      for (int j = 0; j < V; ++j) {
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
          const uint32_t kk = key[j * VEC + q];
          if (kk >= thr) {
            const uint64_t cm = make_comp(kk, elem_idx(j, q));
            if (cm >= prefix) sh.cand[p2++] = cm;
          }
        }
      }
      __syncthreads();
      total = sh.cnt;
      __syncthreads();
    }

    if (total > kRefresh) {
      // cut to the exact top-k so far; later elements need a strictly larger key
      block_select(sh, total);
      for (int i = tid; i < k; i += kNT) sh.cand[i] = sh.list[i];
      if (tid == 0) sh.cnt = k;
      const uint32_t kth = comp_key(sh.list[k - 1]);
      __syncthreads();
      total = k;
      thr = kth + 1u;
    }
    base = total;
#pragma unroll
    for (int j = 0; j < V; ++j) cur[j] = nxt[j];
  }

  block_select(sh, base);
  if (a.nseg == 1) {
    finalize_row<DT, SAMPLE>(a, row, sh.list);
  } else {
    uint64_t* dst = a.ws_lists + ((size_t)row * a.nseg + seg) * kRun;
    for (int i = tid; i < kRun; i += kNT) dst[i] = sh.list[i];
  }
}

// ---------------------------------------------------------------------------
// Kernel B: one wave per row merges the segment lists and finishes the row.
// ---------------------------------------------------------------------------
template <int DT, bool SAMPLE>
__global__ __launch_bounds__(kWave) void seg_merge_kernel(SelArgs a) {
  __shared__ uint64_t list[kRun];
  const int64_t row = blockIdx.x;
  const int l = lane_id();
  const uint64_t* src = a.ws_lists + (size_t)row * a.nseg * kRun;
  uint64_t acc[2] = {src[l], src[kWave + l]};
  for (int s = 1; s < a.nseg; ++s) {
    const uint64_t b[2] = {src[s * kRun + l], src[s * kRun + kWave + l]};
    wave_merge128_desc(acc, b);
  }
  list[l] = acc[0];
  list[kWave + l] = acc[1];
  __syncthreads();
  finalize_row<DT, SAMPLE>(a, row, list);
}

// Standalone top_p_and_sample (sampling.py:210-269) on already-sorted
// candidates [rows, K], K <= 128: one wave per row.
template <int DT>
__global__ __launch_bounds__(kWave) void top_p_sample_kernel(const void* logits, const int32_t* idx,
                                                             int64_t rows, int K, const uint32_t* rng_key,
                                                             const float* top_p, const float* temperature,
                                                             uint32_t vocab, float replace_f32,
                                                             int64_t dim0_offset, int32_t* out) {
  using T = ElemT<DT>;
  const int64_t row = blockIdx.x;
  const int l = lane_id();
  const char* rowp = (const char*)logits + (size_t)row * K * T::ES;
  float v[2];
  int32_t id[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int p = h * kWave + l;
    v[h] = p < K ? __uint_as_float(T::load_bits(rowp, p)) : 0.0f;
    id[h] = p < K ? idx[row * K + p] : 0;
  }
  const int32_t tok = sample_tail(v, id, K, top_p[row], temperature[row], rng_key[0], rng_key[1],
                                  (uint32_t)(row + dim0_offset), vocab, replace_f32);
  if (l == 0) out[row] = tok;
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct Plan {
  int nseg;
  int64_t vps;
};

// Segments: enough workgroups for ~4 per CU, whole tiles per segment, at
// most kMaxSeg segments per row.
static void plan_rows(int64_t rows, int64_t cols, int dt, Plan* p) {
  const int vec = dt == kF32 ? 4 : 8;
  const int V = dt == kF32 ? kVF32 : kVBF16;
  const int64_t tile = (int64_t)kNT * V;
  const int64_t nv = (cols + 2 * (vec - 1)) / vec;  // covers any row misalignment
  const int64_t tiles = (nv + tile - 1) / tile;
  int64_t nseg = (kTargetBlocks + rows - 1) / rows;
  if (nseg > kMaxSeg) nseg = kMaxSeg;
  if (nseg > tiles) nseg = tiles;
  if (nseg < 1) nseg = 1;
  int64_t vps = (nv + nseg - 1) / nseg;
  vps = (vps + tile - 1) / tile * tile;
  nseg = (nv + vps - 1) / vps;
  p->nseg = (int)nseg;
  p->vps = vps;
}

static size_t ws_bytes_for(int64_t rows, const Plan& p) {
  if (p.nseg <= 1) return 0;
  return (size_t)rows * p.nseg * kRun * sizeof(uint64_t);
}

template <int DT, bool SAMPLE>
static int launch_select(const SelArgs& a, hipStream_t s, const char* what) {
  constexpr int V = DT == kF32 ? kVF32 : kVBF16;
  hipLaunchKernelGGL((seg_select_kernel<DT, V, SAMPLE>), dim3((unsigned)a.nseg, (unsigned)a.rows),
                     dim3(kNT), 0, s, a);
  int st = launch_status(what);
  if (st || a.nseg == 1) return st;
  hipLaunchKernelGGL((seg_merge_kernel<DT, SAMPLE>), dim3((unsigned)a.rows), dim3(kWave), 0, s, a);
  return launch_status(what);
}

static float round_to_bf16(float f) {
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

static int check_common(const void* x, int dt, int64_t rows, int64_t cols) {
  if (!x) { set_error("null input pointer"); return kInvalidArgument; }
  if (dt != kF32 && dt != kBF16) { set_error("dtype %d not supported (f32=0, bf16=1)", dt); return kUnsupported; }
  if (rows < 0 || cols <= 0) { set_error("bad shape [%lld, %lld]", (long long)rows, (long long)cols); return kInvalidArgument; }
  if (rows > 65535) { set_error("rows %lld exceeds grid limit 65535", (long long)rows); return kUnsupported; }
  if (cols >= (int64_t)1 << 31) { set_error("cols must fit int32 indices"); return kInvalidArgument; }
  return kOk;
}

}  // namespace tx

using namespace tx;

extern "C" {

size_t tallax_topk_workspace_size(int64_t rows, int64_t cols, int64_t k, int dtype) {
  Plan p;
  if (k < 1 || k > kMaxK || (dtype != kF32 && dtype != kBF16) || rows < 0 || cols <= 0) return 0;
  plan_rows(rows, cols, dtype, &p);
  return ws_bytes_for(rows, p);
}

int tallax_topk(const void* x, int dtype, int64_t rows, int64_t cols, int64_t k, void* out_vals,
                int32_t* out_idx, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  int st = check_common(x, dtype, rows, cols);
  if (st) return st;
  if (k < 1 || k > kMaxK) { set_error("k=%lld outside [1, %d]", (long long)k, kMaxK); return k > kMaxK ? kUnsupported : kInvalidArgument; }
  if (k > cols) { set_error("k=%lld exceeds row length %lld", (long long)k, (long long)cols); return kInvalidArgument; }
  if (!out_vals || !out_idx) { set_error("null output pointer"); return kInvalidArgument; }
  if (rows == 0) return kOk;
  Plan p;
  plan_rows(rows, cols, dtype, &p);
  const size_t need = ws_bytes_for(rows, p);
  if (workspace_bytes < need || (need && !workspace)) {
    set_error("workspace of %zu bytes is smaller than the %zu required", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  SelArgs a = {};
  a.x = x; a.rows = rows; a.cols = cols; a.k = (int)k;
  a.nseg = p.nseg; a.vps = p.vps;
  a.out_vals = out_vals; a.out_idx = out_idx;
  a.ws_lists = (uint64_t*)workspace;
  return dtype == kF32 ? launch_select<kF32, false>(a, stream, "tallax_topk")
                       : launch_select<kBF16, false>(a, stream, "tallax_topk");
}

size_t tallax_sample_workspace_size(int64_t rows, int64_t vocab, int dtype) {
  return tallax_topk_workspace_size(rows, vocab, kMaxK, dtype);
}

int tallax_fused_topk_topp_sample(const void* logits, int dtype, int64_t rows, int64_t vocab,
                                  const int32_t* top_k, const float* top_p, const float* temperature,
                                  const uint32_t* rng_key, int64_t dim0_offset, double replace_val,
                                  int32_t* out_tokens, void* workspace, size_t workspace_bytes,
                                  hipStream_t stream) {
  int st = check_common(logits, dtype, rows, vocab);
  if (st) return st;
  if (vocab < kMaxK) { set_error("vocab %lld < 128 is not supported by the fused sampler", (long long)vocab); return kUnsupported; }
  if (!top_k || !top_p || !temperature || !rng_key || !out_tokens) { set_error("null pointer argument"); return kInvalidArgument; }
  if (rows == 0) return kOk;
  Plan p;
  plan_rows(rows, vocab, dtype, &p);
  const size_t need = ws_bytes_for(rows, p);
  if (workspace_bytes < need || (need && !workspace)) {
    set_error("workspace of %zu bytes is smaller than the %zu required", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  SelArgs a = {};
  a.x = logits; a.rows = rows; a.cols = vocab; a.k = kMaxK;
  a.nseg = p.nseg; a.vps = p.vps;
  a.ws_lists = (uint64_t*)workspace;
  a.top_k = top_k; a.top_p = top_p; a.temperature = temperature; a.rng_key = rng_key;
  a.dim0_offset = dim0_offset;
  const float rf = (float)replace_val;
  a.replace_f32 = rf;
  a.replace_in_dtype = dtype == kBF16 ? round_to_bf16(rf) : rf;
  a.out_tokens = out_tokens;
  return dtype == kF32 ? launch_select<kF32, true>(a, stream, "tallax_fused_topk_topp_sample")
                       : launch_select<kBF16, true>(a, stream, "tallax_fused_topk_topp_sample");
}

int tallax_top_p_and_sample(const void* topk_logits, int dtype, const int32_t* topk_idx, int64_t rows,
                            int64_t k, const uint32_t* rng_key, const float* top_p,
                            const float* temperature, int64_t vocab_size, double replace_val,
                            int64_t dim0_offset, int32_t* out_tokens, hipStream_t stream) {
  int st = check_common(topk_logits, dtype, rows, k);
  if (st) return st;
  if (k > kMaxK) { set_error("k=%lld > 128 candidates per row is not supported", (long long)k); return kUnsupported; }
  if (!topk_idx || !rng_key || !top_p || !temperature || !out_tokens) { set_error("null pointer argument"); return kInvalidArgument; }
  if (rows == 0) return kOk;
  const float rf = (float)replace_val;
  if (dtype == kF32)
    hipLaunchKernelGGL(top_p_sample_kernel<kF32>, dim3((unsigned)rows), dim3(kWave), 0, stream, topk_logits,
                       topk_idx, rows, (int)k, rng_key, top_p, temperature, (uint32_t)vocab_size, rf,
                       dim0_offset, out_tokens);
  else
    hipLaunchKernelGGL(top_p_sample_kernel<kBF16>, dim3((unsigned)rows), dim3(kWave), 0, stream, topk_logits,
                       topk_idx, rows, (int)k, rng_key, top_p, temperature, (uint32_t)vocab_size, rf,
                       dim0_offset, out_tokens);
  return launch_status("tallax_top_p_and_sample");
}

}  // extern "C"
