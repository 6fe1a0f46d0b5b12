// Wide-candidate sampler for gfx950: the fused top-k / top-p / temperature /
// Gumbel draw of sampling.sample with up to 1024 candidates per row instead
// of the reference's 128.
//
// The reference clamps every row's k to max_k = 128 (sampling.py:283-290,
// top_k.py:438-439), so requests with top_k in (128, 1024] are cut.  This
// entry point is the same algorithm with max_k lifted to K <= 1024:
//   * candidates: the K largest values of the row, value descending, ties to
//     the lowest index (the order of xla_equivalent_sort(descending=True,
//     is_stable=True), sort.py:932-970); values the reference's strict-`>`
//     bins can never admit (NaN, -inf, finfo.min; top_k.py:64,241-243) are
//     reported as finfo(dtype).min;
//   * positions >= top_k[row] replaced by replace_val in the logits dtype
//     (top_k.py:365-369);
//   * top_p_mask over the K candidates (sampling.py:25-62): numerators
//     exp(v - v[0]), their sum as a stride-halving tree over
//     W = max(128, pow2ceil(K)) zero-padded slots, cumsum in 8-position tiles
//     (cumsum.py:21-53 on axis 0), t = #(cumsum < p), threshold v[t] or 0
//     when t == K;
//   * scaled = masked / T plus Gumbel noise on the counter (row * vocab +
//     token) (sampling.py:97-111, sparse_random.py:49-57), argmax with
//     max_arrays' tie rule over max(8, pow2ceil(K)) padded slots
//     (bitonic_top_k.py:43-97), greedy idx[0] when T < 1e-5.
// With K = 128 the tokens are those of tallax_fused_topk_topp_sample.
//
// One 1024-thread workgroup per row:
//   radix select: histograms of the select key's digits [31:21], [20:10] and
//     [9:0] (bf16 keys are fixed by their top 16 bits, so two passes), each
//     pass reading the row again and counting only the elements whose higher
//     digits match the threshold prefix found so far, until the K-th largest
//     key is known (or the crossing bin is taken whole);
//   collect: one more read appends the elements above the threshold and the
//     threshold ties to LDS: all ties when they fit a 2048-record list beside
//     the rest, else the first ones in index order (one workgroup scan per
//     8192-column chunk that holds a tie, until enough are taken);
//   a 2048-record bitonic sort of their composites (key << 32 | ~index),
//     whose first K are the candidates;
//   the sampler tail with one candidate per thread.
// The row is read two (bf16) to four (f32) times; the re-reads of a row just
// streamed are served mostly from the caches.
//
// Rows of whole 16-byte vectors that fit 16 vectors per thread (bf16 up to
// 131072 columns, f32 up to 65536) take a single read first: the vectors stay
// in registers; each lane keeps its four largest vector maxima (integer max
// over the raw bits, which orders non-negative values), each wave takes the
// ceil(K / 16)-th largest of its 256 kept maxima, and L, the smallest of those
// over the 16 waves, has at least K elements at or above it (each counted
// maximum is a distinct vector).  When L is a positive value, every element
// >= L goes to the list; with at most 2048 of them the sort below orders them
// and its first K are the candidates.  Other rows (non-positive bound, NaN
// maxima, more than 2048 elements >= L) take the radix select.
#include <float.h>
#include <math.h>
#include <stdint.h>

#include "tallax_hip.h"
#include "tx_block_sort.h"
#include "tx_common.h"
#include "tx_host.h"
#include "tx_sample.h"
#include "tx_scan.h"

namespace tx {

constexpr int kSwNT = 1024;
constexpr int kSwNW = kSwNT / kWave;
constexpr int kSwMaxK = 1024;           // candidates per row, at most (one per thread)
constexpr int kSwList = 2048;           // collected records, at most (two per thread in the sort)
constexpr int kSwBins = 2048;           // 11-bit digits
constexpr int kSwChunk = kSwNT * 8;     // columns per workgroup step: 8 per thread
constexpr int kSwV = 19;                // register path: 16-byte vectors per thread
constexpr int kSwStage = 128;           // register path: staged vectors per wave

typedef short sw_short2_t __attribute__((ext_vector_type(2)));

// Largest element of a 16-byte vector in the signed integer view of its bits
// (monotone over non-negative values; positive NaNs above +inf).
template <int DT>
__device__ __forceinline__ int32_t sw_vec_smax(uint4 v) {
  if constexpr (DT == kBF16) {
    auto mx = [](uint32_t a, uint32_t b) {
      return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(sw_short2_t, a),
                                                                    __builtin_bit_cast(sw_short2_t, b)));
    };
    const uint32_t m = mx(mx(v.x, v.y), mx(v.z, v.w));
    const int32_t lo = (int16_t)(m & 0xFFFFu), hi = (int16_t)(m >> 16);
    return lo > hi ? lo : hi;
  } else {
    const int32_t a = (int32_t)v.x > (int32_t)v.y ? (int32_t)v.x : (int32_t)v.y;
    const int32_t b = (int32_t)v.z > (int32_t)v.w ? (int32_t)v.z : (int32_t)v.w;
    return a > b ? a : b;
  }
}

struct SwArgs {
  const void* x;
  int64_t rows, cols;
  int k;         // candidates per row (K)
  int vec;       // rows start 16-byte aligned: 8-element vector loads
  const int32_t* top_k;
  const float* top_p;
  const float* temperature;
  const uint32_t* rng_key;
  int64_t dim0_offset;
  float replace_f32;       // top_p_mask's fill (sampling.py:58-60)
  float replace_in_dtype;  // the k mask's fill, rounded to the logits dtype
  int32_t* out_tokens;     // [rows], or null
  int32_t* out_idx;        // [rows, K] candidate columns, or null
  float* out_vals;         // [rows, K] candidate values (f32), or null
};

template <int DT>
__device__ __forceinline__ uint32_t sw_key_at(const char* rowp, int64_t i) {
  if constexpr (DT == kBF16) return select_key(((uint32_t)((const uint16_t*)rowp)[i]) << 16);
  else return select_key(((const uint32_t*)rowp)[i]);
}

// Select keys of columns base .. base+7; returns the mask of those inside the row.
template <int DT>
__device__ __forceinline__ uint32_t sw_load8(const char* rowp, int64_t cols, int64_t base, bool vec,
                                             uint32_t (&k)[8]) {
  if (vec && base + 8 <= cols) {
    if constexpr (DT == kBF16) {
      const uint4 w = *(const uint4*)(rowp + base * 2);
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        k[2 * q] = select_key(ws[q] << 16);
        k[2 * q + 1] = select_key(ws[q] & 0xFFFF0000u);
      }
    } else {
      const uint4 w0 = *(const uint4*)(rowp + base * 4);
      const uint4 w1 = *(const uint4*)(rowp + base * 4 + 16);
      const uint32_t ws[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
      for (int q = 0; q < 8; ++q) k[q] = select_key(ws[q]);
    }
    return 0xFFu;
  }
  uint32_t m = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int64_t i = base + q;
    k[q] = 0u;
    if (i < cols) {
      k[q] = sw_key_at<DT>(rowp, i);
      m |= 1u << q;
    }
  }
  return m;
}

// hist[(key >> dsh) & dmask] += 1 over the row's elements whose key >> fsh
// equals fval (every element when !filt).
template <int DT>
__device__ __forceinline__ void sw_hist(const char* rowp, int64_t cols, bool vec, int nchunks, bool filt,
                                        int fsh, uint32_t fval, int dsh, uint32_t dmask, int* hist) {
#pragma unroll 2
  for (int j = 0; j < nchunks; ++j) {
    const int64_t base = ((int64_t)j * kSwNT + threadIdx.x) * 8;
    uint32_t k[8];
    const uint32_t m = sw_load8<DT>(rowp, cols, base, vec, k);
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (((m >> q) & 1u) && (!filt || (k[q] >> fsh) == fval)) atomicAdd(&hist[(k[q] >> dsh) & dmask], 1);
  }
}

// The bin holding the need-th largest counted element (bins scanned from the
// top; thread t owns bins 2047-2t and 2046-2t).  res = {bin, count in higher
// bins, count in the bin}.  Every thread must call it.
__device__ __forceinline__ void sw_cross(const int* hist, int need, int* red, int* res) {
  const int hi = kSwBins - 1 - 2 * (int)threadIdx.x, lo = hi - 1;
  const int h_hi = hist[hi], h_lo = hist[lo];
  int total;
  const int above = block_exscan<kSwNW>(h_hi + h_lo, red, total);
  if (above < need && need <= above + h_hi + h_lo) {
    if (need <= above + h_hi) {
      res[0] = hi; res[1] = above; res[2] = h_hi;
    } else {
      res[0] = lo; res[1] = above + h_hi; res[2] = h_lo;
    }
  }
  __syncthreads();
}

template <int DT>
__global__ __launch_bounds__(kSwNT) void sample_wide_kernel(SwArgs a) {
  constexpr int ES = DT == kBF16 ? 2 : 4;
  __shared__ int s_hist[kSwBins];
  __shared__ uint64_t s_list[kSwList];
  __shared__ uint64_t s_list2[kSwList + 8];  // register path: the candidates in bucket order (+8: unguarded reads)
  __shared__ int32_t s_wmax[kSwNW];
  __shared__ float s_v[kSwMaxK];
  __shared__ float s_e[kSwMaxK];
  __shared__ float s_tot[kSwMaxK / 8];
  __shared__ float s_carry[kSwMaxK / 8];
  __shared__ int s_red[kSwNW];
  __shared__ int s_res[3];
  __shared__ int s_cnt;
  __shared__ float s_sum;
  __shared__ int32_t s_id0;
  __shared__ uint64_t s_bk[kSwNW];
  __shared__ uint4 s_vst[kSwNW][kSwStage];     // register path: the wave's vectors holding a candidate
  __shared__ uint32_t s_vcol[kSwNW][kSwStage];  // and their first column

  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, l = lane_id(), w = t / kWave;
  const int K = a.k;
  // the row's sampling parameters, loaded while the row streams in
  int row_k = 0;
  float row_p = 0.0f, row_temp = 1.0f;
  if (a.out_tokens) {
    row_k = a.top_k[row];
    row_p = a.top_p[row];
    row_temp = a.temperature[row];
  }
  const char* rowp = (const char*)a.x + (size_t)(row * a.cols) * ES;
  const bool vec = a.vec != 0;
  const int nchunks = (int)((a.cols + kSwChunk - 1) / kSwChunk);

  // --- register path: one read, the elements >= L -----------------------------
  constexpr int VEC = DT == kBF16 ? 8 : 4;
  constexpr int32_t kPosInf = DT == kBF16 ? 0x7F80 : 0x7F800000;  // +inf bits in the signed view
  const int64_t nvec = a.cols / VEC;  // a.vec: the row is whole 16-byte vectors
  bool fast = vec && nvec <= (int64_t)kSwNT * kSwV;  // block-uniform
  if (fast) {
    const uint4* vb = (const uint4*)rowp;
    uint4 raw[kSwV];
#pragma unroll
    for (int j = 0; j < kSwV; ++j) {
      const int64_t v = (int64_t)j * kSwNT + t;
      raw[j] = v < nvec ? load_once(vb + v) : make_uint4(~0u, ~0u, ~0u, ~0u);  // all-ones: -1, below every bound
    }
    if (t == 0) s_cnt = 0;
    // this lane's four largest vector maxima; a positive NaN maximum sends the row to the radix select
    int32_t top[4] = {-1, -1, -1, -1};
    bool nan_max = false;
#pragma unroll
    for (int j = 0; j < kSwV; ++j) {
      int32_t x = sw_vec_smax<DT>(raw[j]);
      nan_max |= x > kPosInf;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool sw = x > top[r];
        const int32_t tv = top[r];
        top[r] = sw ? x : tv;
        x = sw ? tv : x;
      }
    }
    // the wave's q-th largest kept maximum among the non-negative ones (-1 if fewer)
    const int q = (K + kSwNW - 1) / kSwNW;
    auto count_ge = [&](int32_t p) {
      int c = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) c += (int)__popcll(__ballot(top[r] >= p));
      return c;
    };
    int32_t wl = -1;
    if (count_ge(1) >= q) {  // wave-uniform; a bound of +0 would need -0 too: positive bounds only
      // two bits per step: the three probes of a step are independent
      constexpr int kBits = DT == kBF16 ? 15 : 31;  // odd: the top bit alone first
      wl = count_ge(1 << (kBits - 1)) >= q ? (1 << (kBits - 1)) : 0;
#pragma unroll 1
      for (int b = kBits - 3; b >= 0; b -= 2) {
        const int32_t p1 = wl | (1 << b), p2 = wl | (2 << b), p3 = wl | (3 << b);
        const int c1 = count_ge(p1), c2 = count_ge(p2), c3 = count_ge(p3);
        wl = c3 >= q ? p3 : (c2 >= q ? p2 : (c1 >= q ? p1 : wl));
      }
    }
    const int32_t wm = wave_max_i(top[0]);  // the wave's largest vector maximum (signed view)
    if (l == 0) {
      s_red[w] = wl;
      s_wmax[w] = wm;
    }
    for (int i = t; i < kSwBins; i += kSwNT) s_hist[i] = 0;  // the bucket counts of the rank below
    fast = !__syncthreads_or(nan_max);
    int32_t L = s_red[0];
#pragma unroll
    for (int i = 1; i < kSwNW; ++i) L = s_red[i] < L ? s_red[i] : L;
    fast = fast && L >= 1;
    if (fast) {
      const uint32_t span = (uint32_t)(kPosInf - L);  // L <= bits <= +inf
      // pass mask of vector j (bit e: element e is >= L)
      auto pass_mask = [&](const uint4 x) -> uint32_t {
        const uint32_t d[4] = {x.x, x.y, x.z, x.w};
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (DT == kBF16) {
            m |= ((uint32_t)((int32_t)(int16_t)(d[i] & 0xFFFFu) - L) <= span ? 1u : 0u) << (2 * i);
            m |= ((uint32_t)(((int32_t)d[i] >> 16) - L) <= span ? 1u : 0u) << (2 * i + 1);
          } else {
            m |= ((uint32_t)((int32_t)d[i] - L) <= span ? 1u : 0u) << i;
          }
        }
        return m;
      };
      // The vectors holding a candidate (maximum >= L; about one in eight for
      // K = 1024) go to the wave's LDS region in lane order, then each lane
      // takes one staged vector at a time: the pass masks, the wave's pool
      // reservation (one scan, one atomic) and the writes then run over the
      // staged vectors only.  A wave with more than kSwStage of them takes
      // every vector from its registers instead.
      int wcnt = 0;
#pragma unroll
      for (int j = 0; j < kSwV; ++j) {
        const bool f = sw_vec_smax<DT>(raw[j]) >= L;
        const uint64_t b = __ballot(f);
        if (b) {  // wave-uniform
          const int o = wcnt + (int)__popcll(b & ((1ull << l) - 1ull));
          if (f && o < kSwStage) {
            s_vst[w][o] = raw[j];
            s_vcol[w][o] = (uint32_t)(((int64_t)j * kSwNT + t) * VEC);
          }
          wcnt += (int)__popcll(b);
        }
      }
      // elements of x (first column col0) in pass mask m go to the pool from slot pos on
      auto put = [&](const uint4 x, uint32_t m, uint32_t col0, int pos) {
        const uint32_t d[4] = {x.x, x.y, x.z, x.w};
        while (m) {
          const int e = __builtin_ctz(m);
          m &= m - 1u;
          const uint32_t bits = DT == kBF16 ? ((e & 1) ? (d[e >> 1] & 0xFFFF0000u) : (d[e >> 1] << 16)) : d[e];
          // every candidate is a positive finite value: its select key is bits | 2^31
          if (pos < kSwList) s_list[pos] = make_comp(bits | 0x80000000u, col0 + (uint32_t)e);
          ++pos;
        }
      };
      if (wcnt <= kSwStage) {  // wave-uniform
        for (int r0 = 0; r0 < wcnt; r0 += kWave) {
          const int o = r0 + l;
          uint4 x = make_uint4(0u, 0u, 0u, 0u);
          uint32_t col0 = 0u, m = 0u;
          if (o < wcnt) {
            x = s_vst[w][o];
            col0 = s_vcol[w][o];
            m = pass_mask(x);
          }
          int wtot;
          const int pre = wave_exscan_i32(__popc(m), wtot);
          int base = 0;
          if (l == 0 && wtot) base = atomicAdd(&s_cnt, wtot);
          put(x, m, col0, __builtin_amdgcn_readfirstlane(base) + pre);
        }
      } else {
        // one pool reservation per wave: the lane's count over its vectors, one
        // wave scan, one atomic; then the writes
        int c = 0;
        uint32_t pm[(kSwV + 3) / 4] = {};  // the masks, 8 bits per vector (VEC <= 8)
#pragma unroll
        for (int j = 0; j < kSwV; ++j) {
          const uint32_t m = pass_mask(raw[j]);
          pm[j >> 2] |= m << (8 * (j & 3));
          c += __popc(m);
        }
        int wtot;
        const int pre = wave_exscan_i32(c, wtot);
        int base = 0;
        if (l == 0 && wtot) base = atomicAdd(&s_cnt, wtot);
        int pos = __builtin_amdgcn_readfirstlane(base) + pre;
#pragma unroll
        for (int j = 0; j < kSwV; ++j) {
          const uint32_t m = (pm[j >> 2] >> (8 * (j & 3))) & 0xFFu;
          if (!__ballot(m != 0u)) continue;  // wave-uniform
          put(raw[j], m, (uint32_t)(((int64_t)j * kSwNT + t) * VEC), pos);
          pos += __popc(m);
        }
      }
      __syncthreads();
      fast = s_cnt <= kSwList;  // block-uniform; s_cnt >= K always
    }
    if (fast) {
      // bucket rank of the n candidates (keys in [select_key(L), kmax]): one
      // atomic per candidate for its bucket count and slot, a scan, a scatter
      // in bucket order, then each candidate's place = its bucket's start +
      // the larger composites in its bucket; places below K go to s_list.
      const int n = s_cnt;
      const uint32_t lkey = select_key(DT == kBF16 ? (uint32_t)L << 16 : (uint32_t)L);
      int32_t kms = s_wmax[0];
#pragma unroll
      for (int i = 1; i < kSwNW; ++i) kms = s_wmax[i] > kms ? s_wmax[i] : kms;
      const uint32_t kmax = select_key(DT == kBF16 ? (uint32_t)kms << 16 : (uint32_t)kms);  // the row's largest key
      uint64_t c2[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) c2[r] = t + r * kSwNT < n ? s_list[t + r * kSwNT] : 0ull;
      // buckets: key buckets of width 2^kshift (largest keys first); where a
      // key bucket holds one key (bf16 keys step by 2^16), nsub column
      // ranges within it (lowest columns first), so that ties spread out
      const uint32_t range = kmax - lkey;  // every candidate key lies in [lkey, kmax]
      int kshift = DT == kBF16 ? 16 : 0;
      while ((range >> kshift) >= (uint32_t)kSwBins) ++kshift;
      const int nkb = (int)(range >> kshift) + 1;
      int nsub = 1;
      if (kshift == (DT == kBF16 ? 16 : 0))
        while (nkb * nsub * 2 <= kSwBins) nsub *= 2;
      int cbits = 0;
      while (((int64_t)1 << cbits) < a.cols) ++cbits;
      int lsub = 0;
      while ((1 << lsub) < nsub) ++lsub;
      const int csh = cbits > lsub ? cbits - lsub : 0;
      int bk[2], slot[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int i = t + r * kSwNT;
        bk[r] = i < n ? (int)((kmax - comp_key(c2[r])) >> kshift) * nsub + (comp_idx(c2[r]) >> csh) : 0;
        slot[r] = i < n ? atomicAdd(&s_hist[bk[r]], 1) : 0;
      }
      __syncthreads();
      {  // exclusive scan: thread t owns buckets 2t, 2t + 1
        const int h0 = s_hist[2 * t], h1 = s_hist[2 * t + 1];
        int total;
        const int before = block_exscan<kSwNW>(h0 + h1, s_red, total);
        s_hist[2 * t] = before;
        s_hist[2 * t + 1] = before + h0;
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < 2; ++r)
        if (t + r * kSwNT < n) s_list2[s_hist[bk[r]] + slot[r]] = c2[r];
      __syncthreads();
      const int nb = nkb * nsub;
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        if (t + r * kSwNT >= n) continue;
        const int st0 = s_hist[bk[r]];
        if (st0 >= K) continue;  // buckets that start at or past place K are not needed
        const int en0 = bk[r] + 1 < nb ? s_hist[bk[r] + 1] : n;
        int rk = st0;
        for (int i0 = st0; i0 < en0; i0 += 8) {  // 8 LDS reads in flight (the buffer is padded)
          uint64_t x[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) x[u] = s_list2[i0 + u];
#pragma unroll
          for (int u = 0; u < 8; ++u) rk += (i0 + u < en0 && x[u] > c2[r]) ? 1 : 0;
        }
        if (rk < K) s_list[rk] = c2[r];
      }
      __syncthreads();
    }
  }

  // --- radix select of the K-th largest key ---------------------------------
  int need = K;          // elements still to take at or below the prefix
  uint32_t prefix = 0;   // digits found so far
  int tsh = 0;           // threshold compares key >> tsh with prefix
  bool take_all = false; // the crossing bin is taken whole
  constexpr int kPasses = DT == kBF16 ? 2 : 3;
#pragma unroll 1
  for (int ps = 0; ps < (fast ? 0 : kPasses); ++ps) {
    const int bits = ps == 2 ? 10 : 11;
    const int dsh = ps == 0 ? 21 : ps == 1 ? 10 : 0;
    for (int i = t; i < kSwBins; i += kSwNT) s_hist[i] = 0;
    __syncthreads();
    sw_hist<DT>(rowp, a.cols, vec, nchunks, ps > 0, dsh + bits, prefix, dsh, (1u << bits) - 1u, s_hist);
    __syncthreads();
    sw_cross(s_hist, need, s_red, s_res);
    const int bin = s_res[0], above = s_res[1], cnt = s_res[2];
    prefix = (prefix << bits) | (uint32_t)bin;
    need -= above;
    tsh = dsh;
    __syncthreads();  // s_res and s_hist are rewritten by the next pass
    // The crossing bin is taken whole when it is all needed, or when all its
    // elements fit the list beside the K - need above it: the sort then puts
    // its ties in index order and the first K records are kept.
    if (need == cnt || K - need + cnt <= kSwList) {
      take_all = true;
      break;
    }
  }

  // --- collect exactly K elements into LDS ------------------------------------
  if (!fast && t == 0) s_cnt = 0;
  __syncthreads();
  int tie_base = 0;  // threshold ties met so far in index order
#pragma unroll 1
  for (int j = 0; j < (fast ? 0 : nchunks); ++j) {
    const int64_t base = ((int64_t)j * kSwNT + t) * 8;
    uint32_t k[8];
    const uint32_t m = sw_load8<DT>(rowp, a.cols, base, vec, k);
    uint32_t take = 0u, eq = 0u;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const uint32_t kp = k[q] >> tsh;
      const bool in = (m >> q) & 1u;
      take |= (in && kp > prefix ? 1u : 0u) << q;
      eq |= (in && kp == prefix ? 1u : 0u) << q;
    }
    if (take_all) {
      take |= eq;
    } else if (tie_base < need) {  // uniform
      if (__syncthreads_or(eq != 0u)) {
        int total;
        const int before = block_exscan<kSwNW>(__popc(eq), s_red, total);
#pragma unroll
        for (int q = 0; q < 8; ++q)
          if (((eq >> q) & 1u) && tie_base + before + __popc(eq & ((1u << q) - 1u)) < need) take |= 1u << q;
        tie_base += total;
      }
    }
    while (take) {
      const int q = __builtin_ctz(take);
      take &= take - 1u;
      const int pos = atomicAdd(&s_cnt, 1);
      if (pos < kSwList) s_list[pos] = make_comp(k[q], (uint32_t)(base + q));
    }
  }
  __syncthreads();

  // --- sort the K candidates, descending (the register path ranked them) -----
  if (!fast) {
    const int ncol = min(s_cnt, kSwList);  // K, or more when a tie bin was taken whole
    uint64_t pair[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) pair[r] = 2 * t + r < ncol ? s_list[2 * t + r] : 0ull;
    __syncthreads();
    block_bitonic_sort_c<uint64_t, 2, kSwList, true>(pair, s_list);
#pragma unroll
    for (int r = 0; r < 2; ++r) s_list[2 * t + r] = pair[r];
    __syncthreads();
  }
  uint64_t rec[1];
  rec[0] = s_list[t];

  const bool in = t < K;
  const uint32_t kk = comp_key(rec[0]);
  const int32_t id = comp_idx(rec[0]);
  const uint32_t min_bits = DT == kBF16 ? 0xff7f0000u : 0xff7fffffu;  // finfo(dtype).min as f32
  const float val = __uint_as_float(kk > ineligible_key_max(DT) ? key_to_bits(kk) : min_bits);
  if (in && a.out_idx) a.out_idx[row * K + t] = id;
  if (in && a.out_vals) a.out_vals[row * K + t] = val;
  if (!a.out_tokens) return;  // uniform

  // --- top-p mask, temperature, Gumbel-max (no contraction: built with -ffp-contract=off)
  const float vv = t < row_k ? val : a.replace_in_dtype;
  s_v[t] = vv;
  if (t == 0) s_id0 = id;
  // the first candidate's value, as thread 0 has it (s_list is complete)
  const uint32_t kk0 = comp_key(s_list[0]);
  const float val0 = __uint_as_float(kk0 > ineligible_key_max(DT) ? key_to_bits(kk0) : min_bits);
  const float v0 = 0 < row_k ? val0 : a.replace_in_dtype;
  const float e = in ? candidate_exp(vv, v0) : 0.0f;
  s_e[t] = e;
  int W = 128;
  while (W < K) W <<= 1;
  __syncthreads();
  if (t < kWave) {
    // the stride-halving tree over the W slots (slot = slot + slot[+h] for
    // h = W/2 .. 64), slot t + 64 k held in register k of lane t, then the wave
    constexpr int KR = kSwMaxK / kWave;
    float v[KR];
#pragma unroll
    for (int k = 0; k < KR; ++k) v[k] = k * kWave < W ? s_e[t + k * kWave] : 0.0f;
#pragma unroll
    for (int hk = KR / 2; hk >= 1; hk >>= 1) {
      if (hk * kWave < W) {  // uniform
#pragma unroll
        for (int k = 0; k < hk; ++k) v[k] = v[k] + v[k + hk];
      }
    }
    float s = v[0];
#pragma unroll
    for (int d = kWave / 2; d >= 1; d >>= 1) s = s + lane_xor_f(s, d);
    if (t == 0) s_sum = s;
  }
  __syncthreads();
  float c = in ? e / s_sum : 0.0f;
#pragma unroll
  for (int sh = 1; sh < 8; sh <<= 1) {
    const float u = row_shr_f(c, sh);
    c = c + ((l & 7) >= sh ? u : 0.0f);
  }
  const int g = t >> 3;
  const int ntiles = (K + 7) >> 3;
  if ((t & 7) == 7) s_tot[g] = c;
  __syncthreads();
  // the candidate's Gumbel noise: waves 1-15 draw it while thread 0 sums the
  // tile totals, wave 0 after that
  const uint32_t row_ctr = (uint32_t)(row + a.dim0_offset);
  float gn = 0.0f;
  if (t >= kWave && in) gn = candidate_noise(a.rng_key[0], a.rng_key[1], row_ctr, (uint32_t)a.cols, id);
  if (t == 0) {
    // carry_g = t_0 + ... + t_{g-1}, one add after the other in tile order,
    // by one lane (-0 + x == x, so the chain starts exactly at t_0), the
    // totals read from LDS 16 at a time
    float run = -0.0f;
    float cur[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) cur[u] = s_tot[u];
    for (int i0 = 0; i0 < ntiles; i0 += 16) {
      float nxt[16];
      const int n0 = i0 + 16 < kSwMaxK / 8 ? i0 + 16 : i0;  // in bounds; unused past the last batch
#pragma unroll
      for (int u = 0; u < 16; ++u) nxt[u] = s_tot[n0 + u];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        s_carry[i0 + u] = run;
        run = run + cur[u];
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) cur[u] = nxt[u];
    }
  }
  if (t < kWave && in) gn = candidate_noise(a.rng_key[0], a.rng_key[1], row_ctr, (uint32_t)a.cols, id);
  __syncthreads();
  if (in && g != 0) c = c + s_carry[g];
  const int tcount = __syncthreads_count(in && c < row_p);
  const float thr = tcount < K ? s_v[tcount] : 0.0f;

  int P = 8;
  while (P < K) P <<= 1;
  int pbits = 0;
  while ((1 << pbits) < P) ++pbits;
  const float temp = row_temp;
  // One u64 key per slot, as max_arrays orders them: the score as an
  // order-preserving integer (-0 as +0) above the bit-reversed position, so
  // the largest key is the largest score with ties to the largest
  // bit-reversed position; padding slots (K <= t < P) score -FLT_MAX and
  // give INT32_MIN, slots past P get key 0 and never win.
  uint64_t key = 0ull;
  if (t < P) {
    float sc = -FLT_MAX;
    if (in) {
      const float masked = vv >= thr ? vv : a.replace_f32;
      const float scaled = masked / temp;
      sc = scaled + gn;
    }
    uint32_t sb = __float_as_uint(sc);
    sb = sb == 0x80000000u ? 0u : sb;
    const uint32_t ord = sb ^ ((uint32_t)((int32_t)sb >> 31) | 0x80000000u);
    key = ((uint64_t)ord << 32) | bitrev((uint32_t)t, pbits);
  }
  auto reduce = [&]() {
#pragma unroll
    for (int d = kWave / 2; d >= 1; d >>= 1) {
      const uint64_t o = shfl_xor_u64(key, d);
      key = o > key ? o : key;
    }
  };
  reduce();
  if (l == 0) s_bk[w] = key;
  __syncthreads();
  if (t < kWave) {
    key = l < kSwNW ? s_bk[l] : 0ull;
    reduce();
    const int pw = (int)bitrev((uint32_t)key, pbits);  // the winning slot (uniform)
    const int32_t tok = pw < K ? comp_idx(s_list[pw]) : INT32_MIN;
    if (t == 0) a.out_tokens[row] = temp < 1e-5f ? s_id0 : tok;
  }
}

}  // namespace tx

using namespace tx;

extern "C" {

int tallax_sample_wide(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t max_k,
                       const int32_t* top_k, const float* top_p, const float* temperature,
                       const uint32_t* rng_key, int64_t dim0_offset, double replace_val, int32_t* out_tokens,
                       int32_t* out_idx, float* out_vals, hipStream_t stream) {
  if (!logits) { set_error("null input pointer"); return kInvalidArgument; }
  if (dtype != kF32 && dtype != kBF16) { set_error("dtype %d not supported (f32=0, bf16=1)", dtype); return kUnsupported; }
  if (rows < 0 || vocab <= 0) { set_error("bad shape [%lld, %lld]", (long long)rows, (long long)vocab); return kInvalidArgument; }
  if (rows > 0x7FFFFFFF || vocab >= (int64_t)1 << 31) { set_error("shape [%lld, %lld] exceeds int32 rows / columns", (long long)rows, (long long)vocab); return kInvalidArgument; }
  if (max_k < 1 || max_k > kSwMaxK) {
    set_error("max_k=%lld outside [1, %d]", (long long)max_k, kSwMaxK);
    return max_k > kSwMaxK ? kUnsupported : kInvalidArgument;
  }
  if (max_k > vocab) { set_error("max_k=%lld exceeds the vocabulary %lld", (long long)max_k, (long long)vocab); return kInvalidArgument; }
  if (!out_tokens && !out_idx && !out_vals) { set_error("no output requested"); return kInvalidArgument; }
  if (out_tokens && (!top_k || !top_p || !temperature || !rng_key)) { set_error("null sampling parameter pointer"); return kInvalidArgument; }
  if (rows == 0) return kOk;
  SwArgs a = {};
  a.x = logits; a.rows = rows; a.cols = vocab; a.k = (int)max_k;
  const int es = dtype == kBF16 ? 2 : 4;
  a.vec = ((uintptr_t)logits % 16 == 0) && ((vocab * es) % 16 == 0);
  a.top_k = top_k; a.top_p = top_p; a.temperature = temperature; a.rng_key = rng_key;
  a.dim0_offset = dim0_offset;
  const float rf = (float)replace_val;
  a.replace_f32 = rf;
  a.replace_in_dtype = dtype == kBF16 ? round_to_bf16(rf) : rf;
  a.out_tokens = out_tokens; a.out_idx = out_idx; a.out_vals = out_vals;
  if (dtype == kF32)
    sample_wide_kernel<kF32><<<dim3((unsigned)rows), dim3(kSwNT), 0, stream>>>(a);
  else
    sample_wide_kernel<kBF16><<<dim3((unsigned)rows), dim3(kSwNT), 0, stream>>>(a);
  return launch_status("tallax_sample_wide");
}

}  // extern "C"
