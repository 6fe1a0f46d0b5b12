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
//   pass 1 (one streaming read, waves claiming 6 x 64-vector batches from an
//           LDS counter): the row maximum, the exp-sum (online, per thread)
//           and, per 64-byte group of the row, the high 16 bits of the group
//           maximum's select key, kept in LDS with a 256-bin histogram of
//           their top byte;
//   threshold: the k-th largest group prefix q0 (the histogram, then one of
//           the low byte inside the crossing bin).  At least k groups reach
//           q0, so at least k elements have a key >= q0 << 16: that is T0;
//   pass 2: the groups that reach q0 (~k of them for Gaussian rows) are
//           listed, spread evenly over the workgroup and read again; their
//           elements >= T0 are appended to LDS;
// then a bucketed rank sort of the candidates (a bitonic network when a key
// bucket is large), the outputs, the tile scan and the cutoff.  Rows too long
// for the group summary (over 24 Ki groups) keep each thread's four largest
// values in pass 1 instead, take T0 as the k-th largest of those 4096 and
// read the whole row again.  If the candidates overflow (heavy ties), the
// k-th composite is found by bisection over the row instead.
#include <float.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "tallax_hip.h"
#include "tx_block_sort.h"
#include "tx_common.h"
#include "tx_host.h"
#include "tx_scan.h"

namespace tx {

constexpr int kPfNT = 1024;
constexpr int kPfNW = kPfNT / kWave;
constexpr int kPfCapMax = 8192;          // candidate records in LDS, at most
constexpr int kPfDynBytes = 75 * 1024;   // dynamic LDS: two row workgroups (with their static LDS) per CU
constexpr int kPfMaxK = 4096;
constexpr int kPfMaxGroups = 24 * 1024;  // 16-bit group maxima in LDS, 24 per thread at most
constexpr int kPfMaxBatches = kPfMaxGroups * 4 / (6 * 64) + 1;  // wave-batches of pass 1, at most
constexpr int kPfBuckets = 512;          // key buckets of the candidate rank sort
constexpr int kPfRankMax = 128;          // largest bucket the rank sort takes (else bitonic)

struct PfArgs {
  const float* x;
  int64_t rows, cols;
  int k;
  float p;
  int cap;   // candidate records in the LDS pool
  int cap2;  // records that fit the region after the pool
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

// For 256 counters h[] in LDS, the largest bin b whose suffix count
// sum(h[b..255]) is >= need (-1 if none); *above = sum(h[b+1..255]).  One
// whole wave calls it.
__device__ __forceinline__ int pf_crossing_bin(const uint32_t* h, uint32_t need, uint32_t* above) {
  const int l = lane_id();
  const uint4 hv = ((const uint4*)h)[l];  // bins 4l .. 4l + 3
  const uint32_t hs[4] = {hv.x, hv.y, hv.z, hv.w};
  const uint32_t incl = wave_incl_scan(hv.x + hv.y + hv.z + hv.w);
  uint32_t suf = (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1) - incl;  // bins of higher lanes
  int cnt = 0;
#pragma unroll
  for (int j = 3; j >= 0; --j) {
    suf += hs[j];
    cnt += suf >= need ? 1 : 0;
  }
  const int b = wave_sum_i(cnt) - 1;  // suffix counts fall with b: the bins that reach need are 0..b
  uint32_t ab = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) ab += 4 * l + j > b ? hs[j] : 0u;
  *above = (uint32_t)wave_sum_i((int)ab);
  return b;
}

// 8 waves per SIMD: two row workgroups share a CU, so one streams while the
// other sorts.  SUMM: group summary and histogram threshold (rows of at most
// kPfMaxGroups groups); otherwise per-thread top-4 and a full second read.
template <bool SUMM>
__global__ __launch_bounds__(kPfNT) __attribute__((amdgpu_waves_per_eu(8, 8)))
void softmax_topk_kernel(PfArgs a) {
  extern __shared__ __align__(16) uint64_t pool[];  // a.cap records, then the group maxima / list / probabilities
  __shared__ __align__(16) uint32_t hist_all[kPfBuckets];  // the two threshold histograms, later the sort buckets
  uint32_t* hist = hist_all;
  uint32_t* hist2 = hist_all + 256;
  __shared__ float redf[kPfNW];
  __shared__ int redi[kPfNW];
  __shared__ uint32_t s_t0, s_above;
  __shared__ int s_cnt, s_bin, s_next, s_mx;
  __shared__ float s_bmc[kPfMaxBatches], s_bsum[kPfMaxBatches];  // per wave-batch: reference mc, exp-sum
  __shared__ float s_cum_carry[kPfMaxK / 128];
  __shared__ float s_tile_sum[kPfMaxK / 128];
  const int t = threadIdx.x, w = t / kWave, l = lane_id();
  const int64_t row = blockIdx.x;
  const float* xr = a.x + row * a.cols;
  const RowVec<4> rv(xr);
  const int64_t nv = (a.cols + rv.mis + 3) / 4;
  const int k = a.k;
  const int64_t v_lo = rv.mis ? 1 : 0;
  const int64_t v_hi = (a.cols + rv.mis) / 4;  // vectors [v_lo, v_hi) lie wholly inside the row
  const int ngroups = (int)((nv + 3) / 4);     // group g = vectors 4g .. 4g + 3 (SUMM: <= kPfMaxGroups)
  uint16_t* summ = (uint16_t*)(pool + a.cap);
  constexpr float kLog2e = 1.44269504088896341f;
  if (SUMM) {
    if (t < 256) {
      hist[t] = 0u;
      hist2[t] = 0u;
    }
    if (t == 0) s_next = 0;
    __syncthreads();
  }

  // ---- pass 1: maximum, exp-sum, group maxima (or per-thread top-4) ------------
  // The exp-sum is kept per thread as s = sum 2^(x log2 e - mc) for the
  // thread's running maximum m, mc = fl(m log2 e) (0 while m is -inf, so that
  // -inf elements add exactly 0).  When m rises, s is rescaled by 2^(mc_old -
  // mc_new), and at the end by 2^(mc - fl(M log2 e)): the rounding of each mc
  // cancels, so the sum matches the numerators 2^(x log2 e - fl(M log2 e)) of
  // the probabilities even where |M log2 e| is large.  v_max_f32 ignores NaN;
  // a NaN or +inf makes the sum NaN, as it makes jax.nn.softmax NaN.
  float m = -INFINITY, s = 0.0f, mc = 0.0f;
  float top[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  auto raise_max = [&](float vm) {
    if (vm > m) {
      const float mcn = vm * kLog2e;
      s = m == -INFINITY ? s : s * __builtin_amdgcn_exp2f(mc - mcn);  // m = -inf: s is 0 (or NaN)
      m = vm;
      mc = mcn;
    }
  };
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
  // the four values of a vector, dead slots as NaN (ignored by max and by >=)
  auto vec_vals = [&](uint4 q, uint32_t live, float xs[4]) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) xs[i] = __uint_as_float(((live >> i) & 1u) ? d[i] : 0x7FC00000u);
  };
  // maximum over a quad of lanes (the four vectors of a group); all four lanes call it together
  auto group_max = [&](float vm) {
    float gm = fmaxf(vm, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(vm), 0xB1, 0xF, 0xF, false)));
    return fmaxf(gm, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(gm), 0x4E, 0xF, 0xF, false)));
  };
  // lane 0 of a quad, v its vector: the group's 16-bit prefix and its histogram count
  auto put_group = [&](float gm, int64_t v) {
    const uint32_t q16 = select_key(__float_as_uint(gm)) >> 16;
    summ[v >> 2] = (uint16_t)q16;
    atomicAdd(&hist[q16 >> 8], 1u);
  };
  auto top4 = [&](const float xs[4], float vm) {
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
  };
  // any vector (row edges, tail); every thread of the workgroup calls it together
  auto step1 = [&](int64_t v) {
    const uint32_t live = v < nv ? live_mask(v) : 0u;
    const uint4 q = v < nv ? load_once(rv.base + v) : make_uint4(0u, 0u, 0u, 0u);
    float xs[4];
    vec_vals(q, live, xs);
    const float vm = fmaxf(fmaxf(xs[0], xs[1]), fmaxf(xs[2], xs[3]));
    raise_max(vm);
    float vs = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e = pf_exp(xs[i], mc);
      vs += ((live >> i) & 1u) ? e : 0.0f;
    }
    s += vs;
    if constexpr (SUMM) {
      const float gm = group_max(vm);
      if ((l & 3) == 0 && v < nv) put_group(gm, v);
    } else {
      top4(xs, vm);
    }
  };
  // vectors i0 + t + u * kPfNT (u < U), all wholly inside the row
  auto batch1 = [&](int64_t i0, auto u_const) {
    constexpr int U = decltype(u_const)::value;
    uint4 q[U];
#pragma unroll
    for (int u = 0; u < U; ++u) q[u] = load_once(rv.base + i0 + t + u * kPfNT);
    float vm[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      vm[u] = fmaxf(fmaxf(__uint_as_float(q[u].x), __uint_as_float(q[u].y)),
                    fmaxf(__uint_as_float(q[u].z), __uint_as_float(q[u].w)));
    float bm = vm[0];
#pragma unroll
    for (int u = 1; u < U; ++u) bm = fmaxf(bm, vm[u]);
    raise_max(bm);
    float vs[2] = {0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < U; ++u) {
      vs[u & 1] += pf_exp(__uint_as_float(q[u].x), mc);
      vs[u & 1] += pf_exp(__uint_as_float(q[u].y), mc);
      vs[u & 1] += pf_exp(__uint_as_float(q[u].z), mc);
      vs[u & 1] += pf_exp(__uint_as_float(q[u].w), mc);
    }
    s += vs[0] + vs[1];
    if constexpr (SUMM) {
      float gm[U];
#pragma unroll
      for (int u = 0; u < U; ++u) gm[u] = group_max(vm[u]);
      if ((l & 3) == 0) {
#pragma unroll
        for (int u = 0; u < U; ++u) put_group(gm[u], i0 + t + u * kPfNT);
      }
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float xs[4] = {__uint_as_float(q[u].x), __uint_as_float(q[u].y), __uint_as_float(q[u].z),
                             __uint_as_float(q[u].w)};
        top4(xs, vm[u]);
      }
    }
  };
  // SUMM rows: waves claim wave-batches of 6 x 64 vectors (vectors c * 384 +
  // lane + 64 u, all inside the row) from an LDS counter, so that they end
  // pass 1 together; lane j of a quad holds vector j of a group.  Which wave
  // takes which batch varies from run to run, so a batch's exp-sum is formed
  // in the wave (reference mc_c = fl(M_c log2 e) for the batch maximum M_c,
  // lane sums added in a fixed tree) and kept per batch; the batches are
  // merged in batch order at the end, so the row's sum does not depend on
  // the claiming.
  const float ninf = -INFINITY;
  float mb = -INFINITY;  // this lane's maximum over its batches
  auto batchW = [&](int32_t c) {
    constexpr int U = 6;
    const int32_t base = c * (6 * kWave);
    uint4 q[U];
#pragma unroll
    for (int u = 0; u < U; ++u) q[u] = load_once(rv.base + base + l + kWave * u);
    float vm[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      vm[u] = raw_max3(__uint_as_float(q[u].x), __uint_as_float(q[u].y),
                       raw_max3(__uint_as_float(q[u].z), __uint_as_float(q[u].w), ninf));
    float bm = vm[0];
#pragma unroll
    for (int u = 1; u < U; ++u) bm = raw_max(bm, vm[u]);
    mb = raw_max(mb, bm);
    float wm = bm;
#pragma unroll
    for (int d = kWave / 2; d >= 1; d >>= 1) wm = raw_max(wm, lane_xor_f(wm, d));
    const float mcc = wm == -INFINITY ? 0.0f : wm * kLog2e;  // -inf elements add exactly 0
    float vs[2] = {0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < U; ++u) {
      vs[u & 1] += pf_exp(__uint_as_float(q[u].x), mcc);
      vs[u & 1] += pf_exp(__uint_as_float(q[u].y), mcc);
      vs[u & 1] += pf_exp(__uint_as_float(q[u].z), mcc);
      vs[u & 1] += pf_exp(__uint_as_float(q[u].w), mcc);
    }
    const float bsum = wave_sum_f(vs[0] + vs[1]);  // lane 0's value: a fixed order
    if (l == 0) {
      s_bmc[c] = mcc;
      s_bsum[c] = bsum;
    }
    float gm[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float g = raw_max(vm[u], __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(vm[u]), 0xB1, 0xF, 0xF, false)));
      gm[u] = raw_max(g, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(g), 0x4E, 0xF, 0xF, false)));
    }
    if ((l & 3) == 0) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        // select key of the group maximum (never NaN: the maxima start from -inf), -0 as +0
        const uint32_t b = __float_as_uint(gm[u] + 0.0f);
        const uint32_t key = b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
        summ[(base + l + kWave * u) >> 2] = (uint16_t)(key >> 16);
        atomicAdd(&hist[key >> 24], 1u);
      }
    }
  };
  constexpr int kWB = 6 * kWave;  // vectors of a wave-batch
  const int c0 = rv.mis ? 1 : 0;  // the first vector holds elements before the row
  const int cfull = (int)(v_hi / kWB);
  if constexpr (SUMM) {
    for (;;) {
      int c = 0;
      if (l == 0) c = atomicAdd(&s_next, 1);
      c = __builtin_amdgcn_readfirstlane(c) + c0;
      if (c >= cfull) break;
      batchW(c);
    }
    // the rest, in chunks of 64 vectors: [0, 384) when the row starts
    // unaligned, and from the last whole wave-batch to the end
    const int lo_cov = c0 * 6, hi_cov = (cfull > c0 ? cfull : c0) * 6;
    const int h_hi = (int)((nv + kWave - 1) / kWave);
    const int nrest = lo_cov + (h_hi - hi_cov);
    for (int r = w; r < nrest; r += kPfNW) {
      const int h = r < lo_cov ? r : hi_cov + (r - lo_cov);
      step1((int64_t)h * kWave + l);
    }
  } else {
    // the loops are uniform over the workgroup, so quads always see all four lanes
    int64_t i = 0;
    if (rv.mis) {  // the first vector holds elements before the row
      step1(t);
      i = kPfNT;
    }
    for (; i + 6 * kPfNT <= v_hi; i += 6 * kPfNT) batch1(i, std::integral_constant<int, 6>());
    for (; i + kPfNT <= v_hi; i += kPfNT) batch1(i, std::integral_constant<int, 1>());
    for (; i < nv; i += kPfNT) step1(i + t);
  }
  float M = fmaxf(m, mb);
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) M = fmaxf(M, lane_xor_f(M, d));
  if (l == 0) redf[w] = M;
  if constexpr (!SUMM) {
    // threshold: the k-th largest of the 4096 per-thread values (as select keys)
    uint32_t tk[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) tk[r] = select_key(__float_as_uint(top[r]));
    uint32_t* keys = (uint32_t*)pool;
    block_bitonic_sort_c<uint32_t, 4, kPfNT * 4, true>(tk, keys);
    if (t == (k - 1) / 4) s_t0 = tk[(k - 1) % 4];
  }
  if (t == 0) s_cnt = 0;
  __syncthreads();
  M = l < kPfNW ? redf[l] : -INFINITY;
#pragma unroll
  for (int d = kPfNW / 2; d >= 1; d >>= 1) M = fmaxf(M, lane_xor_f(M, d));
  M = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(M)));
  const float mcM = M * kLog2e;
  // the exp-sum: thread sums rescaled to the row maximum (a thread that saw
  // only -inf / dead slots contributes 0, or its NaN)
  s = m == -INFINITY ? s : s * __builtin_amdgcn_exp2f(mc - mcM);
  if constexpr (SUMM) {
    // the wave-batch sums, rescaled the same way, each thread taking batches in a fixed order
    for (int c = c0 + t; c < cfull; c += kPfNT) {
      const float bsum = s_bsum[c];
      s += bsum != 0.0f ? bsum * __builtin_amdgcn_exp2f(s_bmc[c] - mcM) : bsum;
    }
  }

  if constexpr (SUMM) {
    // the k-th largest group prefix: top byte from the histogram, low byte
    // from a histogram of the groups in the crossing bin
    if (w == 0) {
      uint32_t above;
      const int b = pf_crossing_bin(hist, (uint32_t)k, &above);
      if (l == 0) {
        s_bin = b;
        s_above = above;
        s_t0 = 0u;  // fewer than k groups: every element is a candidate
      }
    }
    __syncthreads();
    const int b = s_bin;
    if (b >= 0) {
      for (int g = t; g < ngroups; g += kPfNT) {
        const uint32_t q = summ[g];
        if ((q >> 8) == (uint32_t)b) atomicAdd(&hist2[q & 255u], 1u);
      }
      __syncthreads();
      if (w == 0) {
        uint32_t above2;
        const int b2 = pf_crossing_bin(hist2, (uint32_t)k - s_above, &above2);  // >= 0: hist[b] >= k - above
        if (l == 0) s_t0 = (((uint32_t)b << 8) | (uint32_t)b2) << 16;
      }
      __syncthreads();
    }
  }
  // candidates: key >= T0, i.e. x >= t0f as floats (NaN never passes)
  const float t0f = s_t0 >= 0x007FFFFFu ? __uint_as_float(key_to_bits(s_t0)) : -INFINITY;
  // the threshold histograms are done: their words become the sort's bucket
  // counts (pass 2's barriers order this before the counting)
  if (t < kPfBuckets) hist_all[t] = 0u;

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
  if constexpr (SUMM) {
    // list the groups that reach q0 (in place of the summary: every thread
    // reads its groups before the barrier of the scan, then writes)
    const uint32_t q0 = s_t0 >> 16;
    uint32_t mine = 0;  // bit j: group t + j * kPfNT
    for (int g = t, j = 0; g < ngroups; g += kPfNT, ++j) mine |= (summ[g] >= q0 ? 1u : 0u) << j;
    const int c = __popc(mine);
    const int incl = wave_incl_scan(c);
    if (l == kWave - 1) redi[w] = incl;
    __syncthreads();
    int off = incl - c, nlist = 0;
    for (int i = 0; i < kPfNW; ++i) {
      const int r = redi[i];
      off += i < w ? r : 0;
      nlist += r;
    }
    uint16_t* list = summ;
    while (mine) {
      const int j = __builtin_ctz(mine);
      mine &= mine - 1u;
      list[off++] = (uint16_t)(t + j * kPfNT);
    }
    __syncthreads();
    // quad q reads list entries q, q + 256, ...: lane j of the quad vector j
    // of the group.  Per batch, each lane's candidates get consecutive pool
    // slots from a wave prefix sum and one atomic per wave.
    constexpr int U = 6;
    constexpr int kQuads = kPfNT / 4;
    const int quad = t >> 2, ql = t & 3;
    for (int e0 = 0; e0 < nlist; e0 += U * kQuads) {
      uint4 q[U];
      int32_t vv[U];  // nv < 2^31
#pragma unroll
      for (int j = 0; j < U; ++j) {
        const int e = e0 + quad + j * kQuads;
        vv[j] = e < nlist ? (int32_t)list[e] * 4 + ql : -1;
        if (vv[j] >= nv) vv[j] = -1;  // past the last vector of a partial group
        q[j] = vv[j] >= 0 ? rv.base[vv[j]] : make_uint4(0u, 0u, 0u, 0u);
      }
      uint32_t cm = 0;  // bit 4 j + i: element i of vector j is a candidate
#pragma unroll
      for (int j = 0; j < U; ++j) {
        const uint32_t live = vv[j] >= 0 ? live_mask(vv[j]) : 0u;
        const uint32_t d[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) cm |= (((live >> i) & 1u) && __uint_as_float(d[i]) >= t0f ? 1u : 0u) << (4 * j + i);
      }
      const int c = __popc(cm);
      const int incl = wave_incl_scan(c);
      const int wtot = __builtin_amdgcn_readlane(incl, kWave - 1);
      if (wtot) {
        int base = 0;
        if (l == 0) base = atomicAdd(&s_cnt, wtot);
        int off = __builtin_amdgcn_readfirstlane(base) + incl - c;
#pragma unroll
        for (int j = 0; j < U; ++j) {
          const uint32_t d[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if ((cm >> (4 * j + i)) & 1u) {
              if (off < a.cap) pool[off] = make_comp(select_key(d[i]), (uint32_t)(vv[j] * 4 - rv.mis + i));
              ++off;
            }
          }
        }
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
  // Candidates have keys in [lo, hi] (hi: the row maximum's).  Bucket b
  // holds keys with (hi-side first) offset ((key - lo) >> shift) = 511 - b,
  // so buckets run in descending key order; each candidate's place is its
  // bucket's start plus the number of larger composites in its bucket.
  // Buckets larger than kPfRankMax (ties, near-ties) use the bitonic sort.
  bool ranked = false;
  if (n <= a.cap && n + 8 <= a.cap2) {  // + 8: the rank loop's reads run up to 7 records past a bucket
    const uint32_t lo = s_t0 >= 0x007FFFFFu ? s_t0 : 0x007FFFFFu;
    const uint32_t hi = select_key(__float_as_uint(M));
    const uint32_t range = hi > lo ? hi - lo : 0u;
    const int shift = range >= (uint32_t)kPfBuckets ? 32 - __clz((int)(range / kPfBuckets)) : 0;  // range >> shift < kPfBuckets
    auto bucket = [&](uint64_t c) -> int {
      const uint32_t key = comp_key(c);
      const uint32_t o = key > lo ? (key - lo) >> shift : 0u;
      return kPfBuckets - 1 - (int)(o < (uint32_t)kPfBuckets ? o : (uint32_t)(kPfBuckets - 1));
    };
    uint32_t* bk = hist_all;  // zeroed after the threshold
    for (int i = t; i < n; i += kPfNT) atomicAdd(&bk[bucket(pool[i])], 1u);
    __syncthreads();
    // exclusive scan of the bucket counts and the largest count, by wave 0
    if (w == 0) {
      constexpr int PER = kPfBuckets / kWave;
      uint32_t cnt[PER];
      int loc = 0, mxl = 0;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        cnt[i] = bk[l * PER + i];
        loc += (int)cnt[i];
        mxl = max(mxl, (int)cnt[i]);
      }
      int tot;
      uint32_t run = (uint32_t)wave_exscan_i32(loc, tot);
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        bk[l * PER + i] = run;
        run += cnt[i];
      }
      mxl = wave_max_i(mxl);
      if (l == 0) s_mx = mxl;
    }
    __syncthreads();
    const int mxall = s_mx;
    if (mxall <= kPfRankMax) {
      ranked = true;
      uint64_t* pool2 = (uint64_t*)summ;  // n <= a.cap2 records
      for (int i = t; i < n; i += kPfNT) {
        const uint64_t cc = pool[i];
        pool2[atomicAdd(&bk[bucket(cc)], 1u)] = cc;
      }
      __syncthreads();  // bk[b] is now the end of bucket b
      for (int i = t; i < n; i += kPfNT) {
        const uint64_t cc = pool2[i];
        const int b = bucket(cc);
        const int s0 = b ? (int)bk[b - 1] : 0, e0 = (int)bk[b];
        if (s0 >= k) continue;
        int r = s0;
        for (int j0 = s0; j0 < e0; j0 += 8) {  // 8 LDS reads in flight (the region holds n + 8 records)
          uint64_t x[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) x[u] = pool2[j0 + u];
#pragma unroll
          for (int u = 0; u < 8; ++u) r += (j0 + u < e0 && x[u] > cc) ? 1 : 0;
        }
        if (r < k) pool[r] = cc;
      }
      __syncthreads();
    }
  }
  if (ranked) {
  } else if (n <= a.cap) {
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
    float pr = pf_exp(__uint_as_float(key_to_bits(comp_key(c))), mcM) / s;
    if (row_bad) {
      idx = p;
      pr = NAN;
    }
    probs[p] = pr;
    a.out_probs[row * k + p] = pr;
    a.out_idx[row * k + p] = idx;
  }
  lds_barrier();  // the stores stay in flight
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
  if (w == 0) {
    // the carries in tile order: the totals are read out first (one LDS read
    // per lane), then added one after the other
    const float ts = l < ntiles ? s_tile_sum[l] : 0.0f;
    float acc = 0.0f, mine = 0.0f;
#pragma unroll
    for (int i = 0; i < kPfMaxK / 128; ++i) {
      if (i < ntiles) {  // uniform
        mine = l == i ? acc : mine;
        const float ti = readlane_f(ts, i);
        acc = i == 0 ? ti : add_in_order(acc, ti);
      }
    }
    if (l < ntiles) s_cum_carry[l] = mine;
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
  lds_barrier();
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
  // LDS: the candidate pool, then the group maxima of pass 1 (in place of
  // which pass 2 lists the groups it reads; later the k probabilities).  The
  // pool holds at least 3 Ki records, and the sorts' working set (up to 8 Ki
  // records, 64 KiB) always fits the whole region.
  const int64_t nv_max = (cols + 6) / 4;  // vectors of a row at any alignment
  const int64_t ngroups = (nv_max + 3) / 4;
  const bool summ = ngroups <= kPfMaxGroups;
  const size_t region2 = align_up(summ && ngroups * 2 > (int64_t)k * 4 ? (size_t)ngroups * 2 : (size_t)k * 4, 16);
  int cap = (int)((kPfDynBytes - region2) / 8) / 1024 * 1024;
  if (cap > kPfCapMax) cap = kPfCapMax;
  a.cap = cap;
  a.cap2 = (int)(region2 / 8);
  const size_t lds = (size_t)cap * 8 + region2;
  const hipError_t attr1 = set_dynamic_lds_limit((const void*)softmax_topk_kernel<true>, kPfDynBytes, stream);
  const hipError_t attr0 = set_dynamic_lds_limit((const void*)softmax_topk_kernel<false>, kPfDynBytes, stream);
  if (attr1 != hipSuccess || attr0 != hipSuccess) {
    set_error("hipFuncSetAttribute: %s", hipGetErrorString(attr1 != hipSuccess ? attr1 : attr0));
    return kHipError;
  }
  if (summ)
    hipLaunchKernelGGL(softmax_topk_kernel<true>, dim3((unsigned)rows), dim3(kPfNT), lds, stream, a);
  else
    hipLaunchKernelGGL(softmax_topk_kernel<false>, dim3((unsigned)rows), dim3(kPfNT), lds, stream, a);
  return launch_status("tallax_softmax_topk_cumsum");
}

}  // extern "C"
