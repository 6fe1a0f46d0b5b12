// Prefill-scale softmax -> top-k -> cumsum -> top-p cutoff, fused, for gfx950
// (f32 [1024, 201088], k = 2048, p = 0.9).
//
// The reference composes it from jax.nn.softmax, tax.sort(probs,
// descending=True, return_argsort=True) cut to k (sort.py:768-929), tax.cumsum
// (cumsum.py:32-101) and a count of cumsum < p.  Here, per row:
//   * probs = exp(x - max) / sum(exp(x - max)) (float32; the sum order is this
//     kernel's, so probabilities and their cumsum are pinned to float64 by
//     tolerance, not bit for bit);
//   * the k selected positions are the k largest logits, ties to the lowest
//     index.  Probability is a non-decreasing function of the logit, so this
//     is a descending sort of the probabilities in which equal probabilities
//     keep a valid (the reference's non-stable sort leaves their order open)
//     order, and it is exact;
//   * cumsum over the k sorted probabilities in the reference's tile order
//     (128-position tiles, Hillis-Steele inside, sequential carry);
//   * cutoff = #(cumsum < p).
// A row holding NaN or +inf, or only -inf, gives NaN probabilities (as
// jax.nn.softmax does), indices 0..k-1 and cutoff 0.
//
// One 1024-thread workgroup per row, two workgroups per CU:
//   pass 1 (one streaming read): the row maximum, the exp-sum (online, per
//           thread), each thread's four largest values and, per 64-byte
//           group, the high 16 bits of the group maximum's select key (LDS);
//           the k-th largest of the 4096 per-thread values, T0, has at least
//           k elements >= it;
//   pass 2: only the groups whose maximum can reach T0 are read again, and
//           their elements >= T0 appended to LDS (~k + 4 % for Gaussian rows);
// then a workgroup bitonic sort of the candidates, the outputs, the tile
// scan and the cutoff.  If the candidates overflow (heavy ties), the k-th
// composite is found by bisection over the row instead.
#include <float.h>
#include <math.h>
#include <stdint.h>

#include "tallax_hip.h"
#include "tx_block_sort.h"
#include "tx_common.h"
#include "tx_host.h"
#include "tx_scan.h"

namespace tx {

constexpr int kPfNT = 1024;
constexpr int kPfNW = kPfNT / kWave;
constexpr int kPfCapMax = 8192;        // candidate records in LDS, at most
constexpr int kPfLdsBytes = 80 * 1024;  // two row workgroups per CU
constexpr int kPfMaxK = 4096;

struct PfArgs {
  const float* x;
  int64_t rows, cols;
  int k;
  float p;
  int cap;      // candidate records in the LDS pool
  int use_sum;  // 1: pass 1 writes group maxima, pass 2 re-reads only the groups that can hold candidates
  float* out_probs;
  int32_t* out_idx;
  float* out_cum;
  int32_t* out_cutoff;
};

// exp(x - m) as 2^(x log2 e - m log2 e), mc = m log2 e (v_exp_f32)
__device__ __forceinline__ float pf_exp(float x, float mc) {
  return __builtin_amdgcn_exp2f(__builtin_fmaf(x, 1.44269504088896341f, -mc));
}

template <int E>
__device__ void pf_sort_desc(uint64_t* pool, int n) {
  uint64_t v[E];
  const int t = threadIdx.x;
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int i = t * E + r;
    v[r] = i < n ? pool[i] : 0ull;
  }
  __syncthreads();
  block_bitonic_sort_c<uint64_t, E, kPfNT * E, true>(v, pool);
#pragma unroll
  for (int r = 0; r < E; ++r) pool[t * E + r] = v[r];
  __syncthreads();
}

// 8 waves per SIMD: two row workgroups share a CU, so one streams while the
// other sorts
__global__ __launch_bounds__(kPfNT) __attribute__((amdgpu_waves_per_eu(8, 8)))
void softmax_topk_kernel(PfArgs a) {
  extern __shared__ __align__(16) uint64_t pool[];  // a.cap records, then the group maxima / probabilities
  __shared__ float redf[kPfNW];
  __shared__ int redi[kPfNW];
  __shared__ uint32_t s_t0;
  __shared__ int s_cnt;
  __shared__ float s_cum_carry[kPfMaxK / 128];
  __shared__ float s_tile_sum[kPfMaxK / 128];
  const int t = threadIdx.x, w = t / kWave, l = lane_id();
  const int64_t row = blockIdx.x;
  const float* xr = a.x + row * a.cols;
  const RowVec<4> rv(xr);
  const int64_t nv = (a.cols + rv.mis + 3) / 4;
  const int k = a.k;

  // ---- pass 1: maximum, exp-sum, per-thread top-4 values, group maxima --------
  // The exp-sum is kept per thread relative to the thread's running maximum
  // (rescaled when it rises) and combined at the end.  v_max_f32 ignores NaN;
  // a NaN or +inf makes the sum NaN, as it makes jax.nn.softmax NaN.
  // A group is the 64 bytes (4 vectors) read by one quad of lanes; its
  // maximum, as the high 16 bits of the select key, goes to summ[] so that
  // pass 2 re-reads only groups that can hold an element >= T0.  The loops
  // advance a quad at a time, so the quad exchange always sees all four lanes.
  const int64_t v_lo = rv.mis ? 1 : 0;
  const int64_t v_hi = (a.cols + rv.mis) / 4;  // vectors [v_lo, v_hi) are interior
  uint16_t* summ = (uint16_t*)(pool + a.cap);  // [ceil(nv / 4)] group maxima, later the probabilities
  const bool use_sum = a.use_sum != 0;
  constexpr float kLog2e = 1.44269504088896341f;
  float m = -INFINITY, s = 0.0f;
  float top[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  auto live_mask = [&](int64_t v) -> uint32_t {
    if (v >= v_lo && v < v_hi) return 0xFu;
    uint32_t live = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t e = v * 4 - rv.mis + i;
      live |= (e >= 0 && e < a.cols ? 1u : 0u) << i;
    }
    return live;
  };
  // the four values of a vector, dead slots as NaN (ignored by max and by >)
  auto vec_vals = [&](uint4 q, uint32_t live, float xs[4]) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) xs[i] = __uint_as_float(((live >> i) & 1u) ? d[i] : 0x7FC00000u);
  };
  auto pass1_vec = [&](uint4 q, int64_t v) {
    const uint32_t live = v < nv ? live_mask(v) : 0u;
    float xs[4];
    vec_vals(q, live, xs);
    const float vm = fmaxf(fmaxf(xs[0], xs[1]), fmaxf(xs[2], xs[3]));
    if (vm > m) {
      s = s * __builtin_amdgcn_exp2f((m - vm) * kLog2e);  // m = -inf: s was 0 (or NaN)
      m = vm;
    }
    const float mc = m * kLog2e;
    float vs = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e = xs[i] == -INFINITY ? 0.0f : pf_exp(xs[i], mc);
      vs += ((live >> i) & 1u) ? e : 0.0f;
    }
    s += vs;
    if (vm > top[3]) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float x = xs[i];
        if (x > top[3]) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const bool sw = x > top[r];
            const float tv = top[r];
            top[r] = sw ? x : tv;
            x = sw ? tv : x;
          }
        }
      }
    }
    if (use_sum) {
      float gm = fmaxf(vm, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(vm), 0xB1, 0xF, 0xF, false)));
      gm = fmaxf(gm, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(gm), 0x4E, 0xF, 0xF, false)));
      if ((l & 3) == 0 && v < nv) summ[v >> 2] = (uint16_t)(select_key(__float_as_uint(gm)) >> 16);
    }
  };
  {
    constexpr int U = 6;  // loads in flight per thread
    const int64_t vq = (int64_t)t - (l & 3);  // the quad's first vector
    int64_t i = 0;
    for (; vq + i + (int64_t)(U - 1) * kPfNT + 3 < nv; i += (int64_t)U * kPfNT) {
      uint4 q[U];
#pragma unroll
      for (int u = 0; u < U; ++u) q[u] = rv.base[t + i + u * kPfNT];
#pragma unroll
      for (int u = 0; u < U; ++u) pass1_vec(q[u], t + i + u * kPfNT);
    }
    for (; vq + i < nv; i += kPfNT) {
      const int64_t v = t + i;
      pass1_vec(v < nv ? rv.base[v] : make_uint4(0u, 0u, 0u, 0u), v);
    }
  }
  float M = m;
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) M = fmaxf(M, lane_xor_f(M, d));
  if (l == 0) redf[w] = M;
  // threshold: the k-th largest of the 4096 per-thread values (as select keys)
  uint32_t tk[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) tk[r] = select_key(__float_as_uint(top[r]));
  uint32_t* keys = (uint32_t*)pool;
  block_bitonic_sort_c<uint32_t, 4, kPfNT * 4, true>(tk, keys);
  if (t == (k - 1) / 4) s_t0 = tk[(k - 1) % 4];
  if (t == 0) s_cnt = 0;
  __syncthreads();
  M = redf[0];
  for (int i = 1; i < kPfNW; ++i) M = fmaxf(M, redf[i]);
  const float mc = M * kLog2e;
  // the exp-sum: thread sums rescaled to the row maximum (a thread that saw
  // only -inf / dead slots contributes 0, or its NaN)
  s = m == -INFINITY ? s : s * __builtin_amdgcn_exp2f((m - M) * kLog2e);
  // candidates: x >= T0 as floats (NaN never passes)
  const float t0f = s_t0 >= 0x007FFFFFu ? __uint_as_float(key_to_bits(s_t0)) : -INFINITY;
  const uint16_t q0 = (uint16_t)(s_t0 >> 16);

  // ---- pass 2: candidates ---------------------------------------------------------
  auto pass2_vec = [&](uint4 q, int64_t v) {
    const uint32_t live = live_mask(v);
    float xs[4];
    vec_vals(q, live, xs);
    const float vm = fmaxf(fmaxf(xs[0], xs[1]), fmaxf(xs[2], xs[3]));
    uint32_t mask = 0;
    if (vm >= t0f) {
#pragma unroll
      for (int i = 0; i < 4; ++i) mask |= (xs[i] >= t0f ? 1u : 0u) << i;
    }
    const uint64_t any = __ballot(mask != 0u);
    if (any) {
      for (;;) {
        const bool hc = mask != 0u;
        const uint64_t bm = __ballot(hc);
        if (!bm) break;
        uint64_t c = 0;
        if (hc) {
          const int i = __builtin_ctz(mask);
          mask &= mask - 1u;
          c = make_comp(select_key(__float_as_uint(xs[i])), (uint32_t)(v * 4 - rv.mis + i));
        }
        // one atomic per wave step, issued by the first active lane (lanes
        // may have left the vector loop already)
        const int lead = __builtin_ctzll(__ballot(true));
        int base = 0;
        if (l == lead) base = atomicAdd(&s_cnt, (int)__popcll(bm));
        base = __builtin_amdgcn_readfirstlane(base);
        if (hc) {
          const int off = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bm >> 32),
                                                                __builtin_amdgcn_mbcnt_lo((uint32_t)bm, 0u));
          if (off < a.cap) pool[off] = c;
        }
      }
    }
  };
  __syncthreads();  // the key sort above used the pool
  if (use_sum) {
    // this thread's own vectors t + u * kPfNT (u < 64) in groups that can hold
    // a candidate, re-read in batches of U
    uint64_t todo = 0;
    for (int u = 0; (int64_t)t + (int64_t)u * kPfNT < nv; ++u)
      todo |= (summ[((int64_t)t + (int64_t)u * kPfNT) >> 2] >= q0 ? 1ull : 0ull) << u;
    constexpr int U = 4;
    while (__ballot(todo != 0ull)) {
      uint4 q[U];
      int32_t vv[U];  // nv < 2^31
#pragma unroll
      for (int j = 0; j < U; ++j) {
        vv[j] = -1;
        if (todo) {
          const int u = __builtin_ctzll(todo);
          todo &= todo - 1ull;
          vv[j] = t + u * kPfNT;
          q[j] = rv.base[vv[j]];
        }
      }
#pragma unroll
      for (int j = 0; j < U; ++j) {
        if (__ballot(vv[j] >= 0))
          pass2_vec(vv[j] >= 0 ? q[j] : make_uint4(0x7FC00000u, 0x7FC00000u, 0x7FC00000u, 0x7FC00000u),
                    vv[j] >= 0 ? vv[j] : 0);
      }
    }
  } else {
    constexpr int U = 8;
    int64_t v = t;
    for (; v + (U - 1) * kPfNT < nv; v += U * kPfNT) {
      uint4 q[U];
#pragma unroll
      for (int u = 0; u < U; ++u) q[u] = rv.base[v + u * kPfNT];
#pragma unroll
      for (int u = 0; u < U; ++u) pass2_vec(q[u], v + u * kPfNT);
    }
    for (; v < nv; v += kPfNT) pass2_vec(rv.base[v], v);
  }
  s = wave_sum_f(s);
  __syncthreads();
  if (l == 0) redf[w] = s;
  __syncthreads();
  s = 0.0f;
  for (int i = 0; i < kPfNW; ++i) s += redf[i];
  const int n = s_cnt;
  // NaN or +inf in the row, or a row of -inf only, makes the probabilities NaN,
  // as it makes jax.nn.softmax NaN
  const bool row_bad = s != s || M == -INFINITY;

  // ---- the k largest composites, sorted ---------------------------------------
  if (n <= a.cap) {
    if (n <= kPfNT) pf_sort_desc<1>(pool, n);
    else if (n <= 2 * kPfNT) pf_sort_desc<2>(pool, n);
    else if (n <= 4 * kPfNT) pf_sort_desc<4>(pool, n);
    else pf_sort_desc<8>(pool, n);
  } else {
    // heavy ties: bisection for the k-th largest composite over the row
    uint64_t prefix = 0;
    for (int bit = 63; bit >= 0; --bit) {
      const uint64_t probe = prefix | (1ull << bit);
      int c = 0;
      for (int64_t v = t; v < nv; v += kPfNT) {
        const uint4 q = rv.base[v];
        const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t e = v * 4 - rv.mis + i;
          if (e >= 0 && e < a.cols) c += make_comp(select_key(d[i]), (uint32_t)e) >= probe;
        }
      }
      c = wave_sum_i(c);
      __syncthreads();
      if (l == 0) redi[w] = c;
      __syncthreads();
      int tot = 0;
      for (int i = 0; i < kPfNW; ++i) tot += redi[i];
      if (tot >= k) prefix = probe;
    }
    if (t == 0) s_cnt = 0;
    __syncthreads();
    for (int64_t v = t; v < nv; v += kPfNT) {
      const uint4 q = rv.base[v];
      const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t e = v * 4 - rv.mis + i;
        if (e >= 0 && e < a.cols) {
          const uint64_t c = make_comp(select_key(d[i]), (uint32_t)e);
          if (c >= prefix) pool[atomicAdd(&s_cnt, 1)] = c;  // exactly k <= a.cap of them
        }
      }
    }
    __syncthreads();
    pf_sort_desc<4>(pool, k);
  }

  // ---- probabilities, indices, cumsum, cutoff -----------------------------------
  float* probs = (float*)summ;  // k floats (the group maxima are no longer needed)
  for (int p = t; p < k; p += kPfNT) {
    const uint64_t c = pool[p];
    int32_t idx = comp_idx(c);
    float pr = pf_exp(__uint_as_float(key_to_bits(comp_key(c))), mc) / s;
    if (row_bad) {
      idx = p;
      pr = NAN;
    }
    probs[p] = pr;
    a.out_probs[row * k + p] = pr;
    a.out_idx[row * k + p] = idx;
  }
  __syncthreads();
  const int ntiles = (k + 127) / 128;
  float c[2] = {0.0f, 0.0f};
  const bool has_tile = w < ntiles;
  if (has_tile) {  // wave w scans tile w (k <= 16 tiles of 128 per pass)
    for (int h = 0; h < 2; ++h) {
      const int p = w * 128 + h * kWave + l;
      c[h] = p < k ? probs[p] : 0.0f;
    }
    hs_scan128(c, l);
    if (l == kWave - 1) s_tile_sum[w] = c[1];
  }
  __syncthreads();
  if (t == 0) {
    float acc = 0.0f;
    for (int i = 0; i < ntiles; ++i) {
      s_cum_carry[i] = acc;
      acc = i == 0 ? s_tile_sum[0] : add_in_order(acc, s_tile_sum[i]);
    }
  }
  __syncthreads();
  int below = 0;
  if (has_tile) {
    const float cy = s_cum_carry[w];
    for (int h = 0; h < 2; ++h) {
      const int p = w * 128 + h * kWave + l;
      const float v = w == 0 ? c[h] : add_in_order(c[h], cy);
      if (p < k) {
        a.out_cum[row * k + p] = v;
        below += v < a.p ? 1 : 0;
      }
    }
  }
  below = wave_sum_i(below);
  if (l == 0) redi[w] = below;
  __syncthreads();
  if (t == 0) {
    int tot = 0;
    for (int i = 0; i < kPfNW; ++i) tot += redi[i];
    a.out_cutoff[row] = tot;
  }
}

}  // namespace tx

using namespace tx;

extern "C" {

int tallax_softmax_topk_cumsum(const float* logits, int64_t rows, int64_t cols, int k, float p, float* out_probs,
                               int32_t* out_idx, float* out_cumsum, int32_t* out_cutoff, hipStream_t stream) {
  if (!logits || !out_probs || !out_idx || !out_cumsum || !out_cutoff) { set_error("null pointer argument"); return kInvalidArgument; }
  if (rows < 0 || cols <= 0) { set_error("bad shape [%lld, %lld]", (long long)rows, (long long)cols); return kInvalidArgument; }
  if (k < 1 || k > kPfMaxK || k > 16 * 128) {
    set_error("k=%d outside [1, 2048]", k);
    return k > 2048 ? kUnsupported : kInvalidArgument;
  }
  if (k > cols) { set_error("k=%d exceeds row length %lld", k, (long long)cols); return kInvalidArgument; }
  if (cols >= (int64_t)1 << 31) { set_error("cols must fit int32 indices"); return kInvalidArgument; }
  if (rows == 0) return kOk;
  if (rows > 2147483647) { set_error("too many rows"); return kUnsupported; }
  PfArgs a = {};
  a.x = logits; a.rows = rows; a.cols = cols; a.k = k; a.p = p;
  a.out_probs = out_probs; a.out_idx = out_idx; a.out_cum = out_cumsum; a.out_cutoff = out_cutoff;
  // LDS: the candidate pool, then the group maxima of pass 1 (reused for the k
  // probabilities).  The group maxima need nv / 4 halfwords and one vector per
  // bit of a 64-bit mask per thread; longer rows re-read everything in pass 2.
  const int64_t nv_max = (cols + 6) / 4;
  const int64_t ngroups = (nv_max + 3) / 4;
  bool use_sum = nv_max <= 64 * (int64_t)kPfNT && ngroups * 2 <= 48 * 1024;
  size_t region2 = align_up(use_sum ? (size_t)(ngroups * 2 > k * 4 ? ngroups * 2 : k * 4) : (size_t)k * 4, 16);
  int cap = (int)((kPfLdsBytes - region2) / 8) / 1024 * 1024;
  if (cap > kPfCapMax) cap = kPfCapMax;
  if (use_sum && cap < 4096) {
    use_sum = false;
    region2 = align_up((size_t)k * 4, 16);
    cap = kPfCapMax;
  }
  a.cap = cap;
  a.use_sum = use_sum ? 1 : 0;
  const size_t lds = (size_t)cap * 8 + region2;
  static const hipError_t attr = hipFuncSetAttribute((const void*)softmax_topk_kernel,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, kPfLdsBytes);
  if (attr != hipSuccess) { set_error("hipFuncSetAttribute: %s", hipGetErrorString(attr)); return kHipError; }
  hipLaunchKernelGGL(softmax_topk_kernel, dim3((unsigned)rows), dim3(kPfNT), lds, stream, a);
  return launch_status("tallax_softmax_topk_cumsum");
}

}  // extern "C"
