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
// Design (one HBM pass per element):
//   * A row is split into `nchunks` chunks; one 256-thread workgroup per chunk
//     streams its chunk with 16-byte loads into registers (MAXV vectors per
//     thread), turning every element into a monotone 32-bit select key.
//   * Lower bound L on the chunk's k-th largest key: the k-th largest of the
//     256 per-thread maxima (at least k elements are >= it).  Only elements
//     with key >= L become candidates (about 1.4k of them for iid data).
//   * Candidates (composite u64 = key << 32 | ~index) are rank-selected into a
//     sorted top-k list.  Inputs with too many candidates (heavy ties) take an
//     exact 64-step bisection on the composite key instead.
//   * Chunk lists go to a workspace; the last workgroup of the row (atomic
//     arrival counter, reset by that workgroup) merges them with a wave64
//     bitonic merge-and-discard tree and either writes (values, indices) or
//     runs the sampler tail on the row's sorted top-128.
#include <float.h>
#include <math.h>
#include <string.h>

#include "tallax_hip.h"
#include "tx_common.h"
#include "tx_host.h"
#include "tx_math.h"

namespace tx {

constexpr int kNT = 256;        // threads per workgroup: 4 wave64s
constexpr int kCap = 1024;      // candidate slots per chunk
constexpr int kMaxK = 128;      // the reference's top-k limit (top_k.py:438-439)
constexpr int kMaxChunks = 48;  // chunk lists held in LDS by the merging workgroup

struct RowSelectArgs {
  const void* x;
  int64_t rows, cols, row_stride;  // row_stride in elements
  int k;
  int nchunks;
  int64_t vpc;  // 16-byte vectors per chunk
  // top-k outputs
  void* out_vals;
  int32_t* out_idx;
  // workspace: rows * nchunks * P composites, then rows arrival counters
  uint64_t* ws_lists;
  uint32_t* ws_count;
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

struct SelShared {
  uint32_t tmax[kNT];
  uint64_t list[kMaxK];
  int red[kNT / kWave];
  int cnt;
  uint32_t L;
  int last;
};

extern __shared__ __align__(16) uint64_t s_dyn[];

__device__ __forceinline__ int block_sum(int v, SelShared& sh) {
  v = wave_sum_i(v);
  __syncthreads();
  if (lane_id() == 0) sh.red[threadIdx.x / kWave] = v;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int i = 0; i < kNT / kWave; ++i) t += sh.red[i];
  return t;
}

// Count of entries strictly greater than c in a descending list.
__device__ __forceinline__ int count_greater(const uint64_t* list, int n, uint64_t c) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (list[mid] > c) lo = mid + 1; else hi = mid;
  }
  return lo;
}

// ---------------------------------------------------------------------------
// Wave64 bitonic merge-and-discard of two descending lists of P composites
// (P = 64: one per lane, P = 128: two per lane, element i at lane i % 64,
// register i / 64).  Result: the P largest of A u B, descending, written to A.
// ---------------------------------------------------------------------------
template <int P>
__device__ __forceinline__ void wave_merge_top(uint64_t* A, const uint64_t* B) {
  constexpr int E = P / kWave;
  const int l = lane_id();
  uint64_t c[E];
#pragma unroll
  for (int h = 0; h < E; ++h) {
    const int i = h * kWave + l;
    const uint64_t a = A[i], b = B[P - 1 - i];
    c[h] = a > b ? a : b;
  }
  if (E == 2) {  // stride 64: the two registers of a lane
    const uint64_t hi = c[0] > c[E - 1] ? c[0] : c[E - 1];
    const uint64_t lo = c[0] > c[E - 1] ? c[E - 1] : c[0];
    c[0] = hi;
    c[E - 1] = lo;
  }
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) {
    const bool lower = (l & d) == 0;
#pragma unroll
    for (int h = 0; h < E; ++h) {
      const uint64_t o = shfl_xor_u64(c[h], d);
      const bool keep_max = lower;
      c[h] = keep_max ? (c[h] > o ? c[h] : o) : (c[h] > o ? o : c[h]);
    }
  }
#pragma unroll
  for (int h = 0; h < E; ++h) A[h * kWave + l] = c[h];
}

// ---------------------------------------------------------------------------
// Sampler tail on one row's sorted candidates, executed by one wave.
// v[h], id[h]: f32 value and token index at position p = h*64 + lane, for
// positions p < K (K <= 128).  Restates top_p_and_sample_arrays
// (sampling.py:65-115), top_p_mask (sampling.py:25-62), the (8,128)-tile
// cumsum order (cumsum.py:21-53) and max_arrays' tie rule
// (bitonic_top_k.py:43-97).
// ---------------------------------------------------------------------------
__device__ int32_t sample_tail(const float v_in[2], const int32_t id_in[2], int K, float top_p,
                               float temp, uint32_t k0, uint32_t k1, uint32_t row_ctr,
                               uint32_t vocab, float mask_val) {
#pragma clang fp contract(off)
  const int l = lane_id();
  const bool in[2] = {l < K, l + kWave < K};
  float v[2] = {v_in[0], v_in[1]};
  int32_t id[2] = {id_in[0], id_in[1]};

  // softmax numerators exp(l - l[0]) and their total, summed as a
  // stride-halving tree over 128 zero-padded slots.
  const float l0 = shfl_f(v[0], 0);
  float e[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) e[h] = in[h] ? tx_expf(v[h] - l0) : 0.0f;
  float s = e[0] + e[1];
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) s = s + __shfl_xor(s, d, kWave);

  // inclusive cumsum of probs along the candidate axis: Hillis-Steele inside
  // 8-slot tiles, then the running total of earlier tiles added sequentially.
  float c[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) c[h] = e[h] / s;
#pragma unroll
  for (int sh = 1; sh < 8; sh <<= 1) {
    const bool ok = (l & 7) >= sh;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float u = __shfl_up(c[h], sh, kWave);
      c[h] = c[h] + (ok ? u : 0.0f);
    }
  }
  const int tile0 = l >> 3;  // tile of register 0; register 1 is tile0 + 8
  float carry0 = 0.0f, carry1 = 0.0f;
  float run = __shfl(c[0], 7, kWave);
#pragma unroll
  for (int g = 1; g < 16; ++g) {
    if (tile0 == g) carry0 = run;
    if (tile0 + 8 == g) carry1 = run;
    const float tsg = __shfl(g < 8 ? c[0] : c[1], (g & 7) * 8 + 7, kWave);
    run = run + tsg;
  }
  if (tile0 != 0) c[0] = c[0] + carry0;
  c[1] = c[1] + carry1;

  // threshold index t = #(cumsum < p); threshold value l[t] (0 when t == K,
  // the out-of-range gather of take_along_axis_arrays).
  const int t = __popcll(__ballot(in[0] && c[0] < top_p)) + __popcll(__ballot(in[1] && c[1] < top_p));
  const float vt = __shfl(t < kWave ? v[0] : v[1], t & (kWave - 1), kWave);
  const float thr = t < K ? vt : 0.0f;

  // mask, temperature, Gumbel noise, argmax
  int P = 8;
  while (P < K) P <<= 1;
  int pbits = 0;
  while ((1 << pbits) < P) ++pbits;
  float best_s = 0.0f;
  uint32_t best_b = 0;
  int32_t best_i = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int p = h * kWave + l;
    float sc;
    int32_t tok = id[h];
    if (in[h]) {
      const float masked = v[h] >= thr ? v[h] : mask_val;
      const float scaled = masked / temp;
      uint32_t o0, o1;
      threefry2x32(k0, k1, 0u, row_ctr * vocab + (uint32_t)id[h], o0, o1);
      sc = scaled + gumbel_from_bits(o0 ^ o1);
    } else if (p < P) {
      sc = -FLT_MAX;  // max_arrays pads with finfo.min and iinfo.min payloads
      tok = INT32_MIN;
    } else {
      sc = -INFINITY;
    }
    const uint32_t br = p < P ? bitrev((uint32_t)p, pbits) : 0u;
    if (h == 0 || sc > best_s || (sc == best_s && br > best_b)) {
      best_s = sc;
      best_b = br;
      best_i = tok;
    }
  }
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) {
    const float os = __shfl_xor(best_s, d, kWave);
    const uint32_t ob = (uint32_t)__shfl_xor((int)best_b, d, kWave);
    const int32_t oi = __shfl_xor(best_i, d, kWave);
    if (os > best_s || (os == best_s && ob > best_b)) {
      best_s = os;
      best_b = ob;
      best_i = oi;
    }
  }
  const int32_t greedy = __shfl(id[0], 0, kWave);
  return temp < 1e-5f ? greedy : best_i;
}

// ---------------------------------------------------------------------------
// The row-select kernel.
// ---------------------------------------------------------------------------
template <int DT, int MAXV, int P, bool SAMPLE>
__global__ __launch_bounds__(kNT) void row_select_kernel(RowSelectArgs a) {
  using T = ElemT<DT>;
  constexpr int VEC = T::VEC, ES = T::ES, E = MAXV * VEC;
  __shared__ SelShared sh;
  const int tid = threadIdx.x;
  const int chunk = blockIdx.x;
  const int64_t row = blockIdx.y;
  const int k = a.k;

  const char* rowp = (const char*)a.x + (size_t)(row * a.row_stride) * ES;
  const RowVec<ES> rv(rowp);
  const int64_t nv = (a.cols + rv.mis + VEC - 1) / VEC;
  const int64_t v0 = (int64_t)chunk * a.vpc;
  const int64_t v1 = v0 + a.vpc < nv ? v0 + a.vpc : nv;

  // ---- stream the chunk into registers --------------------------------------
  uint4 raw[MAXV];
#pragma unroll
  for (int j = 0; j < MAXV; ++j) {
    const int64_t v = v0 + (int64_t)j * kNT + tid;
    raw[j] = v < v1 ? rv.base[v] : make_uint4(0u, 0u, 0u, 0u);
  }
  uint32_t key[E];
  uint32_t tmax = 0;
#pragma unroll
  for (int j = 0; j < MAXV; ++j) {
    const int64_t v = v0 + (int64_t)j * kNT + tid;
    const int64_t e0 = v * VEC - rv.mis;
    const bool live = v < v1;
    const bool full = live && e0 >= 0 && e0 + VEC <= a.cols;
#pragma unroll
    for (int q = 0; q < VEC; ++q) {
      const bool ok = full || (live && e0 + q >= 0 && e0 + q < a.cols);
      const uint32_t kq = ok ? select_key(T::bits(raw[j], q)) : 0u;
      key[j * VEC + q] = kq;
      tmax = kq > tmax ? kq : tmax;
    }
  }
  auto elem_idx = [&](int j, int q) -> uint32_t {
    return (uint32_t)((v0 + (int64_t)j * kNT + tid) * VEC + q - rv.mis);
  };

  // ---- lower bound L: k-th largest of the per-thread maxima -----------------
  sh.tmax[tid] = tmax;
  if (tid == 0) sh.cnt = 0;
  __syncthreads();
  {
    int r = 0;
    const uint4* t4 = (const uint4*)sh.tmax;
#pragma unroll 8
    for (int j = 0; j < kNT / 4; ++j) {
      const uint4 q = t4[j];
      const int b = 4 * j;
      r += (q.x > tmax) + ((q.x == tmax) & (b + 0 < tid));
      r += (q.y > tmax) + ((q.y == tmax) & (b + 1 < tid));
      r += (q.z > tmax) + ((q.z == tmax) & (b + 2 < tid));
      r += (q.w > tmax) + ((q.w == tmax) & (b + 3 < tid));
    }
    if (r == k - 1) sh.L = tmax;
  }
  __syncthreads();
  const uint32_t L = sh.L > 1u ? sh.L : 1u;

  // ---- candidates: every live element with key >= L --------------------------
  uint64_t* cand = s_dyn;
  int cnt = 0;
#pragma unroll
  for (int i = 0; i < E; ++i) cnt += key[i] >= L;
  int pos = 0;
  if (cnt > 0) pos = atomicAdd(&sh.cnt, cnt);
  if (cnt > 0 && pos + cnt <= kCap) {
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
#pragma unroll
      for (int q = 0; q < VEC; ++q) {
        if (key[j * VEC + q] >= L) cand[pos++] = make_comp(key[j * VEC + q], elem_idx(j, q));
      }
    }
  }
  __syncthreads();
  int total = sh.cnt;

  if (total > kCap) {
    // Too many candidates (heavy ties at L): find the exact k-th largest
    // composite by bisection over its 64 bits, then keep exactly k elements.
    uint64_t prefix = 0;
    for (int bit = 63; bit >= 0; --bit) {
      const uint64_t probe = prefix | (1ull << bit);
      int c = 0;
#pragma unroll
      for (int j = 0; j < MAXV; ++j) {
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
          const uint32_t kk = key[j * VEC + q];
          c += (kk != 0u) && make_comp(kk, elem_idx(j, q)) >= probe;
        }
      }
      if (block_sum(c, sh) >= k) prefix = probe;
    }
    __syncthreads();
    if (tid == 0) sh.cnt = 0;
    __syncthreads();
    int c = 0;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
#pragma unroll
      for (int q = 0; q < VEC; ++q) {
        const uint32_t kk = key[j * VEC + q];
        c += (kk != 0u) && make_comp(kk, elem_idx(j, q)) >= prefix;
      }
    }
    int p2 = c > 0 ? atomicAdd(&sh.cnt, c) : 0;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
#pragma unroll
      for (int q = 0; q < VEC; ++q) {
        const uint32_t kk = key[j * VEC + q];
        if (kk != 0u) {
          const uint64_t cc = make_comp(kk, elem_idx(j, q));
          if (cc >= prefix) cand[p2++] = cc;
        }
      }
    }
    __syncthreads();
    total = sh.cnt;
  }

  // ---- rank-select the chunk's sorted top-k (zero-padded to P) ---------------
  for (int i = tid; i < P; i += kNT) sh.list[i] = 0;
  __syncthreads();
  for (int i = tid; i < total; i += kNT) {
    const uint64_t c = cand[i];
    int r = 0;
    int j = 0;
    for (; j + 2 <= total; j += 2) {
      const uint64_t a0 = cand[j], a1 = cand[j + 1];
      r += (a0 > c) + (a1 > c);
    }
    if (j < total) r += cand[j] > c;
    if (r < k) sh.list[r] = c;
  }
  __syncthreads();

  const uint64_t* final_list = sh.list;
  if (a.nchunks > 1) {
    uint64_t* dst = a.ws_lists + ((size_t)row * a.nchunks + chunk) * P;
    for (int i = tid; i < P; i += kNT) dst[i] = sh.list[i];
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const uint32_t old = atomicAdd(&a.ws_count[row], 1u);
      sh.last = old == (uint32_t)(a.nchunks - 1);
    }
    __syncthreads();
    if (!sh.last) return;
    __threadfence();
    if (tid == 0) a.ws_count[row] = 0u;  // ready for the next launch
    const uint64_t* src = a.ws_lists + (size_t)row * a.nchunks * P;
    uint64_t* lists = s_dyn;
    for (int i = tid; i < a.nchunks * P; i += kNT) lists[i] = src[i];
    __syncthreads();
    const int wave = tid / kWave;
    for (int stride = 1; stride < a.nchunks; stride <<= 1) {
      for (int i = 2 * stride * wave; i + stride < a.nchunks; i += 2 * stride * (kNT / kWave)) {
        wave_merge_top<P>(lists + (size_t)i * P, lists + (size_t)(i + stride) * P);
      }
      __syncthreads();
    }
    final_list = lists;
  }

  // ---- outputs ---------------------------------------------------------------
  const uint32_t inel = ineligible_key_max(DT);
  if (!SAMPLE) {
    for (int i = tid; i < k; i += kNT) {
      const uint64_t c = final_list[i];
      const uint32_t kk = comp_key(c);
      const int32_t idx = comp_idx(c);
      const uint32_t b = kk > inel ? T::load_bits(rowp, idx) : T::kMinBits;
      T::store(a.out_vals, row * k + i, b);
      a.out_idx[row * k + i] = idx;
    }
  } else if (tid < kWave) {
    const int l = lane_id();
    const int kr = a.top_k[row];
    float v[2];
    int32_t id[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int p = h * kWave + l;
      const uint64_t c = final_list[p];
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
  int maxv;
  int nchunks;
  int64_t vpc;
  int P;
};

static const int kMaxvF32[] = {2, 4, 8, 16};
static const int kMaxvBF16[] = {1, 2, 4, 8};

// Chunking policy: the largest per-thread register tile that still gives at
// least 2048 workgroups (8 per CU) over the whole launch; small launches use
// the smallest tile to spread rows over as many CUs as possible.  A chunk has
// at least 256 vectors so that every thread holds live data.
static int plan_rows(int64_t rows, int64_t cols, int k, int dt, Plan* p) {
  const int vec = dt == kF32 ? 4 : 8;
  const int64_t nv = (cols + 2 * (vec - 1)) / vec;  // covers any row misalignment
  const int* opts = dt == kF32 ? kMaxvF32 : kMaxvBF16;
  p->P = k <= 64 ? 64 : 128;
  int chosen = -1;
  for (int o = 3; o >= 0; --o) {
    const int64_t per = (int64_t)kNT * opts[o];
    const int64_t nch = (nv + per - 1) / per;
    if (nch <= kMaxChunks && rows * nch >= 2048) { chosen = o; break; }
  }
  if (chosen < 0) {
    for (int o = 0; o < 4; ++o) {
      const int64_t per = (int64_t)kNT * opts[o];
      if ((nv + per - 1) / per <= kMaxChunks) { chosen = o; break; }
    }
  }
  if (chosen < 0) {
    set_error("row length %lld exceeds the %d-chunk limit of this build", (long long)cols, kMaxChunks);
    return kUnsupported;
  }
  p->maxv = opts[chosen];
  const int64_t per = (int64_t)kNT * p->maxv;
  int64_t nch = (nv + per - 1) / per;
  // balance: spread vectors evenly, keeping >= kNT vectors per chunk
  int64_t vpc = (nv + nch - 1) / nch;
  if (vpc < kNT) vpc = kNT;
  nch = (nv + vpc - 1) / vpc;
  p->nchunks = (int)nch;
  p->vpc = vpc;
  return kOk;
}

static size_t ws_bytes_for(int64_t rows, const Plan& p) {
  if (p.nchunks <= 1) return 0;
  return align_up((size_t)rows * p.nchunks * p.P * sizeof(uint64_t), 256) +
         align_up((size_t)rows * sizeof(uint32_t), 256);
}

template <int DT, int MAXV, int P, bool SAMPLE>
static void launch_one(const RowSelectArgs& a, hipStream_t s) {
  const size_t lds = sizeof(uint64_t) * (size_t)(a.nchunks * P > kCap ? a.nchunks * P : kCap);
  dim3 grid((unsigned)a.nchunks, (unsigned)a.rows);
  hipLaunchKernelGGL((row_select_kernel<DT, MAXV, P, SAMPLE>), grid, dim3(kNT), lds, s, a);
}

template <int DT, bool SAMPLE>
static void launch_dt(const RowSelectArgs& a, const Plan& p, hipStream_t s) {
  constexpr bool F = DT == kF32;
  const int m = p.maxv;
  if (p.P == 64) {
    if (SAMPLE) return;  // the sampler always selects 128 candidates
    if (m == (F ? 2 : 1)) launch_one<DT, F ? 2 : 1, 64, false>(a, s);
    else if (m == (F ? 4 : 2)) launch_one<DT, F ? 4 : 2, 64, false>(a, s);
    else if (m == (F ? 8 : 4)) launch_one<DT, F ? 8 : 4, 64, false>(a, s);
    else launch_one<DT, F ? 16 : 8, 64, false>(a, s);
  } else {
    if (m == (F ? 2 : 1)) launch_one<DT, F ? 2 : 1, 128, SAMPLE>(a, s);
    else if (m == (F ? 4 : 2)) launch_one<DT, F ? 4 : 2, 128, SAMPLE>(a, s);
    else if (m == (F ? 8 : 4)) launch_one<DT, F ? 8 : 4, 128, SAMPLE>(a, s);
    else launch_one<DT, F ? 16 : 8, 128, SAMPLE>(a, s);
  }
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
  if (k < 1 || k > kMaxK || (dtype != kF32 && dtype != kBF16)) return 0;
  if (plan_rows(rows, cols, (int)k, dtype, &p) != kOk) return 0;
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
  st = plan_rows(rows, cols, (int)k, dtype, &p);
  if (st) return st;
  const size_t need = ws_bytes_for(rows, p);
  if (workspace_bytes < need || (need && !workspace)) {
    set_error("workspace of %zu bytes is smaller than the %zu required", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  RowSelectArgs a = {};
  a.x = x; a.rows = rows; a.cols = cols; a.row_stride = cols; a.k = (int)k;
  a.nchunks = p.nchunks; a.vpc = p.vpc;
  a.out_vals = out_vals; a.out_idx = out_idx;
  if (need) {
    a.ws_lists = (uint64_t*)workspace;
    a.ws_count = (uint32_t*)((char*)workspace + align_up((size_t)rows * p.nchunks * p.P * sizeof(uint64_t), 256));
  }
  if (dtype == kF32) launch_dt<kF32, false>(a, p, stream);
  else launch_dt<kBF16, false>(a, p, stream);
  return launch_status("tallax_topk");
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
  st = plan_rows(rows, vocab, kMaxK, dtype, &p);
  if (st) return st;
  const size_t need = ws_bytes_for(rows, p);
  if (workspace_bytes < need || (need && !workspace)) {
    set_error("workspace of %zu bytes is smaller than the %zu required", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  RowSelectArgs a = {};
  a.x = logits; a.rows = rows; a.cols = vocab; a.row_stride = vocab; a.k = kMaxK;
  a.nchunks = p.nchunks; a.vpc = p.vpc;
  if (need) {
    a.ws_lists = (uint64_t*)workspace;
    a.ws_count = (uint32_t*)((char*)workspace + align_up((size_t)rows * p.nchunks * p.P * sizeof(uint64_t), 256));
  }
  a.top_k = top_k; a.top_p = top_p; a.temperature = temperature; a.rng_key = rng_key;
  a.dim0_offset = dim0_offset;
  const float rf = (float)replace_val;
  a.replace_f32 = rf;
  a.replace_in_dtype = dtype == kBF16 ? round_to_bf16(rf) : rf;
  a.out_tokens = out_tokens;
  if (dtype == kF32) launch_dt<kF32, true>(a, p, stream);
  else launch_dt<kBF16, true>(a, p, stream);
  return launch_status("tallax_fused_topk_topp_sample");
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
