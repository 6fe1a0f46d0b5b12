// Binned top-k for gfx950: tax.top_dynamic_k, with guarantee_convergence's
// bin-packing merge of unconverged blocks (binned_merge_kernel).
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
//     truncated to max_k, with replace_val at positions >= k[row];
//   * a block writes only the ranks of the steps it evaluated: ranks at or
//     past the m of its last evaluated step keep the finfo.min the scratch
//     starts with (top_k.py:241-243, 250-281), so they count as fillers in
//     the final selection even where depth_upper reaches past them.
// The ranks inside a bin are the same whatever the pass structure (each pass
// extends the exact per-bin top-m), so one scan computes the deepest lists
// and every step's statistics; the select kernel drops the ranks a block
// never evaluated.
//
// Kernels:
//   binned_lists_kernel  one workgroup per row: thread (bin, slice) scans
//                        every S-th element of its bin keeping a register
//                        top-MC list; the slices of a bin are merged through
//                        LDS; ranks < buf go to the workspace with each
//                        step's (pivot, count).
//   binned_finish_kernel one workgroup: depths, cutoffs, valid, depth_upper
//                        and each row's last evaluated m.
//   binned_merge_kernel  one workgroup per row of an unconverged block
//                        (guarantee_convergence, last depth != max_k):
//                        the busiest bins packed whole into rank 0.
//   binned_select_kernel one workgroup per row: bitonic sort of the
//                        depth_upper * num_bins superset, top-128 out.
#include <float.h>
#include <stdint.h>
#include <string.h>

#include "tallax_hip.h"
#include "tallax_hip_testing.h"
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
  float replace_val;       // in the input dtype (float inputs)
  int32_t replace_i;       // int32 inputs: replace_val converted with saturation
  int merge;               // bin-packing merge of unconverged blocks
  int num_packed;          // bins packed by the merge (a power of two <= 128)
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
  int32_t* row_fc;         // [rows] first converged step (nsteps if none)
  int32_t* blk_last;       // [rows / block_token] last step each block evaluated
  int32_t* row_mlast;      // [rows] m of the last step the row's block evaluated
  // candidate path
  const uint64_t* lists;   // [rows][nseg][128] per-segment sorted top-128 composites
  int nseg;
  int32_t* covered;        // [rows] 1: the candidates settled the row, 0: it was scanned
};

__device__ __forceinline__ float load_val(const void* x, int dt, int64_t i) {
  return dt == kBF16 ? __uint_as_float(((uint32_t)((const uint16_t*)x)[i]) << 16) : ((const float*)x)[i];
}
__device__ __forceinline__ float dtype_min_f(int dt) {
  return dt == kBF16 ? __uint_as_float(0xFF7F0000u) : -FLT_MAX;
}

// The 32-bit values the per-bin lists hold: float for float32 and bfloat16
// inputs (bfloat16 widened), int32 for int32 inputs.  The lists only compare,
// take maxima of and move values, so one template covers both; the workspace
// arrays are 32-bit either way.
//   lowest    the dtype's min, where bins start (finfo.min / iinfo.min,
//             top_k.py:241-243 via utils.py:48-56); only strictly greater
//             values are admitted (top_k.py:64)
//   pad       value of a slot past the row: never admitted
//   key       the unsigned select key (monotone, 0 = nothing below it)
//   fill      what the bin-packing merge writes into a chosen bin: the min of
//             the 32-bit scratch dtype (top_k.py:147-151)
template <typename VT>
struct BinVal;
template <>
struct BinVal<float> {
  static constexpr bool kInt = false;
  static __device__ __forceinline__ float load(const void* x, int dt, int64_t i) { return load_val(x, dt, i); }
  static __device__ __forceinline__ float lowest(int dt) { return dtype_min_f(dt); }
  static __device__ __forceinline__ float pad() { return -INFINITY; }
  static __device__ __forceinline__ float vmax(float a, float b) { return fmaxf(a, b); }
  static __device__ __forceinline__ uint32_t key(float v) { return select_key(__float_as_uint(v)); }
  static __device__ __forceinline__ float from_key(uint32_t k) { return __uint_as_float(key_to_bits(k)); }
  static __device__ __forceinline__ float fill() { return -FLT_MAX; }
  static __device__ __forceinline__ uint32_t bits(float v) { return __float_as_uint(v); }
  static __device__ __forceinline__ float from_bits(uint32_t u) { return __uint_as_float(u); }
};
template <>
struct BinVal<int32_t> {
  static constexpr bool kInt = true;
  static __device__ __forceinline__ int32_t load(const void* x, int, int64_t i) { return ((const int32_t*)x)[i]; }
  static __device__ __forceinline__ int32_t lowest(int) { return INT32_MIN; }
  static __device__ __forceinline__ int32_t pad() { return INT32_MIN; }
  static __device__ __forceinline__ int32_t vmax(int32_t a, int32_t b) { return a > b ? a : b; }
  static __device__ __forceinline__ uint32_t key(int32_t v) { return (uint32_t)v ^ 0x80000000u; }
  static __device__ __forceinline__ int32_t from_key(uint32_t k) { return (int32_t)(k ^ 0x80000000u); }
  static __device__ __forceinline__ int32_t fill() { return INT32_MIN; }
  static __device__ __forceinline__ uint32_t bits(int32_t v) { return (uint32_t)v; }
  static __device__ __forceinline__ int32_t from_bits(uint32_t u) { return (int32_t)u; }
};

// (value desc, index asc) order: a before b
template <typename VT>
__device__ __forceinline__ bool ahead(VT va, int32_t ia, VT vb, int32_t ib) {
  return va > vb || (va == vb && (uint32_t)ia < (uint32_t)ib);
}

// Full scan of one row by a kBinNT-thread workgroup; smem holds
// kBinNT * MC * 8 bytes.
template <int MC, typename VT>
__device__ __forceinline__ void scan_row(const BinArgs& a, int64_t row, unsigned char* smem) {
  using B = BinVal<VT>;
  const int NB = a.num_bins;
  const int S = kBinNT / NB;  // slices per bin
  VT* sv = (VT*)smem;                               // [S][MC][NB]
  int32_t* si = (int32_t*)(sv + (size_t)S * MC * NB);
  VT* lv = (VT*)a.lv;
  __shared__ VT red_f[kBinNT / kWave];
  __shared__ int red_i[kBinNT / kWave];
  const int t = threadIdx.x;
  const int b = t % NB, s = t / NB;
  const VT lo = B::lowest(a.dtype);
  VT v[MC];
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
    VT xs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = jb + (int64_t)u * step;
      xs[u] = j < a.cols ? B::load(a.x, a.dtype, base + j) : B::pad();
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      VT x = xs[u];
      if (x > v[MC - 1]) {  // strict: ties keep the earlier (lower) index; NaN never enters
        int32_t xi = (int32_t)(jb + (int64_t)u * step);
#pragma unroll
        for (int r = 0; r < MC; ++r) {
          const bool sw = x > v[r];
          const VT tv = v[r];
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
    lv[((size_t)row * a.buf + r) * NB + b] = lo;
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
      const VT cv = sv[((size_t)q * MC + h) * NB + b];
      ++nreal;
#pragma unroll
      for (int r = 0; r < MC; ++r) rank[r] += ahead(cv, ci, v[r], id[r]) ? 1 : 0;
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < MC; ++r) {
    if (id[r] >= 0 && rank[r] < a.buf) {
      lv[((size_t)row * a.buf + rank[r]) * NB + b] = v[r];
      a.li[((size_t)row * a.buf + rank[r]) * NB + b] = id[r];
    }
  }
  // statistics of every schedule step from the ranked entries
  const int w = t / kWave, l = lane_id();
  constexpr int NW = kBinNT / kWave;
  const int kept = nreal < MC ? nreal : MC;  // real entries in the bin's merged list
  for (int q = 0; q < a.nsteps; ++q) {
    const int m = a.steps[q];
    VT pv = B::pad();
#pragma unroll
    for (int r = 0; r < MC; ++r)
      if (id[r] >= 0 && rank[r] == m - 1) pv = B::vmax(pv, v[r]);
    if (s == 0 && kept < m) pv = B::vmax(pv, lo);  // the bin's m-th entry is a filler
    pv = B::vmax(pv, B::from_bits(lane_xor(B::bits(pv), 32)));
    pv = B::vmax(pv, B::from_bits(lane_xor(B::bits(pv), 16)));
    pv = B::vmax(pv, B::from_bits(lane_xor(B::bits(pv), 8)));
    pv = B::vmax(pv, B::from_bits(lane_xor(B::bits(pv), 4)));
    pv = B::vmax(pv, B::from_bits(lane_xor(B::bits(pv), 2)));
    pv = B::vmax(pv, B::from_bits(lane_xor(B::bits(pv), 1)));
    if (l == 0) red_f[w] = pv;
    __syncthreads();
    VT pivot = red_f[0];
    for (int i = 1; i < NW; ++i) pivot = B::vmax(pivot, red_f[i]);
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
      ((VT*)a.st_pivot)[row * a.nsteps + q] = pivot;
      a.st_count[row * a.nsteps + q] = tot;
    }
    __syncthreads();
  }
}

template <int MC, typename VT>
__global__ __launch_bounds__(kBinNT) void binned_lists_kernel(BinArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  scan_row<MC, VT>(a, blockIdx.x, smem);
}

// Depths, cutoffs, valid, depth_upper and each row's last evaluated m from
// the per-step statistics: a row's depth is m - 1 at its first converged step
// (max_k if none); a block of block_token rows evaluates steps until all of
// its rows converged, and its cutoff is the pivot of the last step evaluated.
// Three passes over rows, blocks and rows (any block_token); the barriers
// between them order this workgroup's own global writes and reads.
constexpr int kFinishNT = 1024;

__device__ __forceinline__ int first_converged(const BinArgs& a, int64_t r) {
  const int kr = a.k_rows[r];
  int fc = a.nsteps;
  for (int q = a.nsteps - 1; q >= 0; --q)
    if (a.st_count[r * a.nsteps + q] >= kr) fc = q;
  return fc;
}

__device__ __forceinline__ int depth_upper_of(const BinArgs& a, int g) {
  int up = a.gsched[a.ngs - 1];
  for (int i = 0; i + 1 < a.ngs; ++i) {
    if (a.gsched[i] < g && g <= a.gsched[i + 1]) {
      up = a.gsched[i + 1];
      break;
    }
  }
  return up;
}

__device__ __forceinline__ void finish_rows(const BinArgs& a) {
  __shared__ int red[kFinishNT / kWave];
  const int t = threadIdx.x;
  int gmax = 0;
  for (int64_t r = t; r < a.rows; r += kFinishNT) {
    const int fc = first_converged(a, r);
    a.row_fc[r] = fc;
    const int depth = fc < a.nsteps ? a.steps[fc] - 1 : a.max_k;
    a.out_depths[r] = depth;
    gmax = max(gmax, depth);
  }
  __syncthreads();
  const int64_t nblk = a.rows / a.block_token;
  for (int64_t b = t; b < nblk; b += kFinishNT) {
    int qb = 0;
    for (int64_t i = 0; i < a.block_token; ++i) qb = max(qb, a.row_fc[b * a.block_token + i]);
    a.blk_last[b] = qb < a.nsteps - 1 ? qb : a.nsteps - 1;
  }
  __syncthreads();
  for (int64_t r = t; r < a.rows; r += kFinishNT) {
    const int last = a.blk_last[r / a.block_token];
    ((uint32_t*)a.out_cutoff)[r] = ((const uint32_t*)a.st_pivot)[r * a.nsteps + last];  // float or int32 bits
    a.row_mlast[r] = a.steps[last];
  }
  const int l = lane_id();
  gmax = wave_max_i(gmax);
  if (l == 0) red[t / kWave] = gmax;
  __syncthreads();
  if (t == 0) {
    int g = 0;
    for (int i = 0; i < kFinishNT / kWave; ++i) g = max(g, red[i]);
    a.out_valid[0] = (g < a.steps[a.nsteps - 1] || a.steps[a.nsteps - 1] == a.max_k) ? 1 : 0;
    a.upper[0] = depth_upper_of(a, g);
  }
}

__global__ __launch_bounds__(kFinishNT) void binned_finish_kernel(BinArgs a) { finish_rows(a); }

// ---------------------------------------------------------------------------
// Candidate path.  The segment kernel of the exact top-k gives every segment's
// sorted top-128 composites (value descending, index ascending).  With T0 the
// largest of the segments' 128th composites, every element whose composite is
// >= T0 is among them, since it is >= its own segment's 128th composite.  So
// the set C = {candidates >= T0} is complete, and per bin the
// entries of C are the bin's largest ones, ranked exactly as in the reference's
// per-bin lists.  A row is settled from C when
//   * every schedule step's pivot (the max over bins of the m-th largest) is
//     the m-th entry of some bin of C with a key strictly above T0's, so that
//     every element >= the pivot is in C (and bins with fewer than m entries in
//     C have their m-th largest below it);
//   * no bin overflows its LDS bucket;
//   * at least max_k entries of C sit at ranks below min(depth, buf), so the
//     final top-max_k of the first depth_upper ranks of every bin (depth_upper
//     >= depth) are all in C.
// Its per-bin lists are then written with the ranks C leaves open as fillers,
// which rank below every entry the final selection can return.  Other rows
// are left to the full scan.
// ---------------------------------------------------------------------------
constexpr int kCandNT = 1024;
constexpr int kCandLdsBytes = 128 * 1024;
constexpr int kCandRank = 16;  // ranks kept per bin (>= buf and every step depth)

// Per bin: a bucket of cap entries and a ranked list of min(cap, kCandRank)
// entries, each padded by one entry so that lanes reading their own bins
// spread over the LDS banks, plus a counter.
__host__ __device__ inline size_t cand_bin_bytes(int cap) {
  const int ec = cap < kCandRank ? cap : kCandRank;
  return (size_t)(cap + 1) * 8 + (size_t)(ec + 1) * 8 + 4;
}
__host__ __device__ inline int cand_bucket_cap(int nb) {
  int c = 32;
  while (c > 1 && (size_t)nb * cand_bin_bytes(c) > (size_t)kCandLdsBytes) --c;
  return c;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) {
    const uint64_t o = shfl_xor_u64(v, d);
    v = o > v ? o : v;
  }
  return v;
}

// One workgroup per row (thread t handles bin t for the per-bin steps).  A row
// the candidates do not settle is scanned in full by the same workgroup.
template <int MC>
__global__ __launch_bounds__(kCandNT) void binned_cand_kernel(BinArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NW = kCandNT / kWave;
  const int NB = a.num_bins;
  const int BC = cand_bucket_cap(NB);
  const int EC = BC < kCandRank ? BC : kCandRank;
  const int BS = BC + 1, ES = EC + 1;               // padded strides
  uint64_t* bucket = (uint64_t*)smem;               // [NB][BS]
  uint64_t* ranked = bucket + (size_t)NB * BS;      // [NB][ES]
  int* cnt = (int*)(ranked + (size_t)NB * ES);      // [NB]
  __shared__ unsigned long long s_t0;
  __shared__ unsigned long long s_red64[kMaxSteps][NW];
  __shared__ int s_redi[kMaxSteps][NW];
  __shared__ unsigned long long s_piv[kMaxSteps];
  __shared__ int s_cnt[kMaxSteps];
  __shared__ int s_bad, s_nd;
  const int t = threadIdx.x, w = t / kWave, l = lane_id();
  const int64_t row = blockIdx.x;
  const int n = a.nseg * 128;
  const uint64_t* lst = a.lists + (size_t)row * n;
  const uint32_t inel = ineligible_key_max(a.dtype);
  for (int b = t; b < NB; b += kCandNT) cnt[b] = 0;
  if (t == 0) s_bad = 0;
  // every candidate of the row is loaded at once (n <= 32 * 128 = 4 * kCandNT)
  constexpr int U = 4;
  uint64_t c[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int e = u * kCandNT + t;
    c[u] = e < n ? lst[e] : 0ull;
  }
  if (w == 0) {  // T0: the largest of the segments' 128th composites (nseg <= 64)
    const uint64_t v = wave_max_u64(l < a.nseg ? lst[l * 128 + 127] : 0ull);
    if (l == 0) s_t0 = v;
  }
  __syncthreads();
  const uint64_t t0 = s_t0;
  int bin[U], pos[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    pos[u] = -1;
    bin[u] = 0;
    if (c[u] != 0ull && c[u] >= t0 && comp_key(c[u]) > inel) {
      bin[u] = (int)((uint32_t)comp_idx(c[u]) % (uint32_t)NB);
      pos[u] = atomicAdd(&cnt[bin[u]], 1);
      if (pos[u] < BC) bucket[(size_t)bin[u] * BS + pos[u]] = c[u];
    }
  }
  __syncthreads();
  // rank of each entry inside its bin's bucket
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (pos[u] < 0 || pos[u] >= BC) continue;
    const int nb = cnt[bin[u]] < BC ? cnt[bin[u]] : BC;
    const uint64_t* bk = bucket + (size_t)bin[u] * BS;
    int r = 0;
    for (int j0 = 0; j0 < nb; j0 += 8) {  // 8 LDS reads in flight per batch
      uint64_t x[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = j0 + j < nb ? bk[j0 + j] : 0ull;
#pragma unroll
      for (int j = 0; j < 8; ++j) r += x[j] > c[u] ? 1 : 0;
    }
    if (r < EC) ranked[(size_t)bin[u] * ES + r] = c[u];
  }
  __syncthreads();
  // per-step pivot: the largest m-th entry over bins (thread t = bin t; only
  // the waves holding bins take part in the per-bin steps)
  const int nbw = (NB + kWave - 1) / kWave;
  const bool bw = w < nbw;
  const bool hb = t < NB;
  const int cb_raw = hb ? cnt[t] : 0;
  const int cb = cb_raw < EC ? cb_raw : EC;
  uint32_t rk[kCandRank];
  if (bw) {
    if (__ballot(cb_raw > BC) && l == 0) s_bad = 1;
    for (int q = 0; q < a.nsteps; ++q) {
      const int m = a.steps[q];
      const uint64_t v = wave_max_u64((hb && m <= EC && cb >= m) ? ranked[(size_t)t * ES + m - 1] : 0ull);
      if (l == 0) s_red64[q][w] = v;
    }
#pragma unroll
    for (int i = 0; i < kCandRank; ++i) rk[i] = (hb && i < cb) ? comp_key(ranked[(size_t)t * ES + i]) : 0u;
  }
  __syncthreads();
  if (t < a.nsteps) {
    uint64_t v = 0ull;
    for (int i = 0; i < nbw; ++i) v = s_red64[t][i] > v ? s_red64[t][i] : v;
    s_piv[t] = v;
  }
  __syncthreads();
  // per-step count: entries of ranks < m - 1 with a value >= the pivot
  if (bw) {
    for (int q = 0; q < a.nsteps; ++q) {
      const uint32_t pk = comp_key((uint64_t)s_piv[q]);
      const int lim = a.steps[q] - 1 < cb ? a.steps[q] - 1 : cb;
      int cq = 0;
#pragma unroll
      for (int i = 0; i < kCandRank; ++i) cq += (i < lim && rk[i] >= pk) ? 1 : 0;
      cq = wave_sum_i(cq);
      if (l == 0) s_redi[q][w] = cq;
    }
  }
  __syncthreads();
  if (t < a.nsteps) {
    int v = 0;
    for (int i = 0; i < nbw; ++i) v += s_redi[t][i];
    s_cnt[t] = v;
  }
  __syncthreads();
  // coverage of the steps, the row's depth and the entries below min(depth, buf)
  bool ok = s_bad == 0;
  int depth = a.max_k;
  bool conv = false;
  for (int q = 0; q < a.nsteps; ++q) {
    const uint64_t pv = s_piv[q];
    ok = ok && pv != 0ull && comp_key(pv) > comp_key(t0);
    if (!conv && s_cnt[q] >= a.k_rows[row]) {
      conv = true;
      depth = a.steps[q] - 1;
    }
  }
  // The final selection reads ranks below R = min(depth_upper, m of the last
  // step the row's block evaluated).  A converged row has R >= depth
  // (depth_upper >= min(global max depth, last bucket) >= depth, and its
  // block ran at least to its converging step m = depth + 1); an unconverged
  // row's block ran every step, so R >= min(max_k, m_final - 1).  max_k
  // entries of C below that bound make the final top-max_k come from C.
  const int mf = a.steps[a.nsteps - 1];
  int dm = conv ? depth : (a.max_k < mf - 1 ? a.max_k : mf - 1);
  dm = dm < a.buf ? dm : a.buf;
  if (bw) {
    const int v = wave_sum_i(cb < dm ? cb : dm);
    if (l == 0) s_redi[0][w] = v;
  }
  __syncthreads();
  if (t == 0) {
    int v = 0;
    for (int i = 0; i < nbw; ++i) v += s_redi[0][i];
    s_nd = v;
  }
  __syncthreads();
  ok = ok && s_nd >= a.max_k && dm <= EC;
  if (t == 0) a.covered[row] = ok ? 1 : 0;
  if (ok) {
    if (t < a.nsteps) {
      a.st_pivot[row * a.nsteps + t] = __uint_as_float(key_to_bits(comp_key((uint64_t)s_piv[t])));
      a.st_count[row * a.nsteps + t] = s_cnt[t];
    }
    const float lo = dtype_min_f(a.dtype);
    for (int e = t; e < a.buf * NB; e += kCandNT) {
      const int r = e / NB, b = e % NB;
      const int cbb = cnt[b] < EC ? cnt[b] : EC;
      float v = lo;
      int32_t id = -1;
      if (r < cbb) {
        const uint64_t x = ranked[(size_t)b * ES + r];
        v = __uint_as_float(key_to_bits(comp_key(x)));
        id = comp_idx(x);
      }
      a.lv[((size_t)row * a.buf + r) * NB + b] = v;
      a.li[((size_t)row * a.buf + r) * NB + b] = id;
    }
  } else {
    __syncthreads();  // the scan reuses the LDS
    scan_row<MC, float>(a, row, smem);
  }
}

__host__ __device__ inline size_t cand_lds_bytes(int nb) { return (size_t)nb * cand_bin_bytes(cand_bucket_cap(nb)); }

// composite of a list entry: value descending then index ascending as an
// unsigned number, so that a scratch filler (finfo.min, index -1) follows
// every entry of its value or above with a real index; 0 stays "no entry"
template <typename VT>
__device__ __forceinline__ uint64_t entry_comp(VT v, int32_t i) {
  return make_comp(BinVal<VT>::key(v), (uint32_t)i);
}

// float -> bfloat16 bits, nearest even (NaN kept quiet): list values are
// bfloat16 values except the merge's float32 finfo.min, which becomes -inf
__device__ __forceinline__ uint16_t bf16_bits_rne(float v) {
  const uint32_t b = __float_as_uint(v);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b | 0x00400000u) >> 16);
  return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

// Binary-tree merge of the sorted top-128 lists held by waves 0..nwr-1
// (acc, two entries per lane) through LDS; wave 0 ends with the merged list.
// Every thread of the workgroup must call it.
template <int NW>
__device__ __forceinline__ void tree_merge128(uint64_t acc[2], int nwr, uint64_t (*tree)[128]) {
  const int w = (int)(threadIdx.x / kWave), l = lane_id();
  for (int st = 1; st < nwr; st <<= 1) {
    if ((w & (2 * st - 1)) == st) {
      tree[w][l] = acc[0];
      tree[w][kWave + l] = acc[1];
    }
    __syncthreads();
    if ((w & (2 * st - 1)) == 0 && w + st < nwr) {
      const uint64_t b[2] = {tree[w + st][l], tree[w + st][kWave + l]};
      wave_merge128_desc(acc, b);
    }
  }
}

// Top max_k of the first depth_upper ranks of every bin: each wave sorts
// 128-entry runs of the superset (wave64 bitonic network) and folds them into
// its own top-128 by merge-and-discard; the per-wave lists are merged as a
// binary tree through LDS.
// With INLINE (rows <= kFinishNT), every workgroup first recomputes the
// finish step for all rows (a few values per row) to get depth_upper, and
// writes its own row's depth and cutoff (workgroup 0 also `valid`), which
// saves a kernel launch; otherwise binned_finish_kernel ran before.
constexpr int kSelNT = 1024;
static_assert(kSelNT == kFinishNT, "the inline finish step uses one thread per row");
template <bool INLINE, typename VT>
__global__ __launch_bounds__(kSelNT) void binned_select_kernel(BinArgs a) {
  using B = BinVal<VT>;
  constexpr int NW = kSelNT / kWave;
  __shared__ uint64_t tree[NW][128];
  __shared__ int fcs[kSelNT];
  __shared__ int red[NW];
  __shared__ int s_mlast;
  const int t = threadIdx.x, w = t / kWave, l = lane_id();
  const int64_t row = blockIdx.x;
  const int NB = a.num_bins;
  // this wave's 128-entry runs of all buf ranks are loaded before depth_upper is known
  constexpr int kPre = 2;  // runs per wave prefetched
  const int nall = a.buf * NB;
  const VT* lv = (const VT*)a.lv + (size_t)row * a.buf * NB;  // rank-major: entry e = rank * NB + bin
  const int32_t* li = a.li + (size_t)row * a.buf * NB;
  VT pv[kPre][2];
  int32_t pi[kPre][2];
#pragma unroll
  for (int k = 0; k < kPre; ++k) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int e = (w + k * NW) * 128 + h * kWave + l;
      pv[k][h] = e < nall ? lv[e] : (VT)0;
      pi[k][h] = e < nall ? li[e] : -1;
    }
  }
  int upper_v, mlast;
  if (INLINE) {
    const bool live = t < a.rows;
    const int fc = live ? first_converged(a, t) : a.nsteps;
    fcs[t] = fc;
    int g = live ? (fc < a.nsteps ? a.steps[fc] - 1 : a.max_k) : 0;
    g = wave_max_i(g);
    if (l == 0) red[w] = g;
    __syncthreads();
    g = 0;
    for (int i = 0; i < NW; ++i) g = max(g, red[i]);
    upper_v = depth_upper_of(a, g);
    if (t == 0) {
      // rows <= kSelNT and block_token divides rows, so the block lies in fcs
      const int r = (int)row;
      const int b0 = r / a.block_token * a.block_token;
      int qb = 0;
      for (int i = 0; i < a.block_token; ++i) qb = max(qb, fcs[b0 + i]);
      const int last = qb < a.nsteps - 1 ? qb : a.nsteps - 1;
      const int fr = fcs[r];
      a.out_depths[row] = fr < a.nsteps ? a.steps[fr] - 1 : a.max_k;
      ((uint32_t*)a.out_cutoff)[row] = ((const uint32_t*)a.st_pivot)[row * a.nsteps + last];
      if (row == 0) a.out_valid[0] = (g < a.steps[a.nsteps - 1] || a.steps[a.nsteps - 1] == a.max_k) ? 1 : 0;
      s_mlast = a.steps[last];
    }
    __syncthreads();
    mlast = s_mlast;
  } else {
    upper_v = a.upper[0];
    mlast = a.row_mlast[row];
  }
  // ranks the row's block never evaluated stay fillers
  const int up0 = upper_v < a.buf ? upper_v : a.buf;
  const int up = up0 < mlast ? up0 : mlast;
  const int n = up * NB;
  const int nr = (n + 127) / 128;
  uint64_t acc[2] = {0ull, 0ull};
  for (int r = w; r < nr; r += NW) {
    uint64_t c[2];
    const int k = (r - w) / NW;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int e = r * 128 + h * kWave + l;
      if (k < kPre) {
        c[h] = e < n ? entry_comp(k == 0 ? pv[0][h] : pv[1][h], k == 0 ? pi[0][h] : pi[1][h]) : 0ull;
      } else {
        c[h] = e < n ? entry_comp(lv[e], li[e]) : 0ull;
      }
    }
    wave_sort128_desc(c);
    if (r == w) {
      acc[0] = c[0];
      acc[1] = c[1];
    } else {
      wave_merge128_desc(acc, c);
    }
  }
  tree_merge128<NW>(acc, nr < NW ? nr : NW, tree);  // waves holding a list
  if (w != 0) return;
  const VT lo = B::lowest(a.dtype);
  const int kr = a.k_rows[row];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int p = h * kWave + l;
    if (p >= a.max_k) continue;
    const uint64_t c = acc[h];
    VT v = lo;
    int32_t id = -1;
    if (c != 0ull) {
      v = B::from_key(comp_key(c));
      id = comp_idx(c);
    }
    const int64_t o = row * a.max_k + p;
    if constexpr (B::kInt) {
      ((int32_t*)a.out_vals)[o] = (a.has_replace && p >= kr) ? a.replace_i : (int32_t)v;
    } else {
      if (a.has_replace && p >= kr) v = a.replace_val;
      if (a.dtype == kBF16)
        ((uint16_t*)a.out_vals)[o] = bf16_bits_rne(v);
      else
        ((float*)a.out_vals)[o] = v;
    }
    a.out_idx[o] = id;
  }
}

// ---------------------------------------------------------------------------
// Bin-packing merge of the blocks that did not converge, for
// guarantee_convergence with a last depth m other than max_k
// (_merge_unconverged_bins_top_k, top_k.py:108-200, invoked at :317-331).
// One workgroup per row, after the finish step; rows of converged blocks
// return at once.
//   1. per bin b, cnt[b] = #(ranks < m-1 whose value is >= the last step's
//      pivot); the P bins of the largest counts are chosen (equal counts:
//      lowest bin first), by a wave sort of (cnt, bin) composites;
//   2. the packed entries (position e < npk: column (e / P) * NB +
//      chosen[e % P], or (finfo.min, that column) past the row's end) and
//      rank 0 of bins 0..127 (float32's finfo.min for chosen bins) are
//      reduced to their top 128: each wave sorts 128-entry runs and merges
//      them into its list, skipping runs with nothing above its 128th
//      entry, then the waves' lists are merged;
//   3. rank 0 of bins 0..127 takes that top 128, and every other rank of a
//      chosen bin takes float32's finfo.min with its index kept.
// ---------------------------------------------------------------------------
constexpr int kMergeNT = 1024;
static_assert(kMergeNT >= kBinNT, "one thread per bin");
template <typename VT>
__global__ __launch_bounds__(kMergeNT) void binned_merge_kernel(BinArgs a) {
  using B = BinVal<VT>;
  constexpr int NW = kMergeNT / kWave;
  __shared__ uint64_t tree[NW][128];
  __shared__ int s_chosen[128];
  __shared__ unsigned char s_isch[kBinNT];
  const int t = threadIdx.x, w = t / kWave, l = lane_id();
  const int64_t row = blockIdx.x;
  const int NB = a.num_bins, P = a.num_packed;
  const int last = a.nsteps - 1;
  const int m = a.steps[last];
  const int64_t b0 = row / a.block_token * a.block_token;
  int open = 0;
  for (int64_t i = t; i < a.block_token; i += kMergeNT) open |= a.row_fc[b0 + i] >= a.nsteps ? 1 : 0;
  if (!__syncthreads_or(open)) return;  // the block converged
  VT* lv = (VT*)a.lv + (size_t)row * a.buf * NB;  // rank-major: entry rank * NB + bin
  int32_t* li = a.li + (size_t)row * a.buf * NB;
  const VT pivot = ((const VT*)a.st_pivot)[row * a.nsteps + last];
  // 1. counts, as (count, bin) composites in LDS, then the top 128 of them
  uint64_t* cb = &tree[0][0];  // NB <= NW * 128 entries
  if (t < NB) {
    int c = 0;
    for (int i = 0; i < m - 1; ++i) c += lv[(size_t)i * NB + t] >= pivot ? 1 : 0;
    cb[t] = make_comp((uint32_t)c, (uint32_t)t);
    s_isch[t] = 0;
  }
  __syncthreads();
  const int nbr = (NB + 127) / 128;
  uint64_t acc[2] = {0ull, 0ull};
  if (w < nbr) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int e = w * 128 + h * kWave + l;
      acc[h] = e < NB ? cb[e] : 0ull;
    }
    wave_sort128_desc(acc);
  }
  __syncthreads();  // the tree reuses the counts' LDS
  tree_merge128<NW>(acc, nbr, tree);
  if (w == 0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int p = h * kWave + l;
      if (p < P) {
        const int b = comp_idx(acc[h]);
        s_chosen[p] = b;
        s_isch[b] = 1;
      }
    }
  }
  __syncthreads();
  // 2. top 128 of the packed entries and rank 0 of bins 0..127
  const int64_t V = a.cols;
  const int64_t npk = (V + (int64_t)128 * (NB / P) - 1) / ((int64_t)128 * (NB / P)) * 128;
  const int64_t nr = npk / 128 + 1;  // runs; the last one is rank 0 of bins 0..127
  const VT lo = B::lowest(a.dtype);
  const uint32_t lo_key = B::key(lo);
  const int64_t xrow = row * V;
  auto entry = [&](int64_t e) -> uint64_t {
    if (e < npk) {
      const int64_t col = (e / P) * NB + s_chosen[e % P];
      const uint32_t key = col < V ? B::key(B::load(a.x, a.dtype, xrow + col)) : lo_key;
      return make_comp(key, (uint32_t)col);
    }
    const int c = (int)(e - npk);
    return entry_comp<VT>(s_isch[c] ? B::fill() : lv[c], li[c]);
  };
  constexpr int U = 4;  // runs loaded per batch
  acc[0] = acc[1] = 0ull;
  bool have = false;
  for (int64_t r0 = w; r0 < nr; r0 += (int64_t)U * NW) {
    uint64_t c[U][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t r = r0 + (int64_t)u * NW;
#pragma unroll
      for (int h = 0; h < 2; ++h) c[u][h] = r < nr ? entry(r * 128 + h * kWave + l) : 0ull;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (r0 + (int64_t)u * NW >= nr) break;
      if (have) {
        const uint64_t a1 = acc[1];
        const uint64_t thr = ((uint64_t)readlane_u32((uint32_t)(a1 >> 32), kWave - 1) << 32) |
                             readlane_u32((uint32_t)a1, kWave - 1);
        if (!__any(c[u][0] > thr || c[u][1] > thr)) continue;
      }
      wave_sort128_desc(c[u]);
      if (!have) {
        acc[0] = c[u][0];
        acc[1] = c[u][1];
        have = true;
      } else {
        wave_merge128_desc(acc, c[u]);
      }
    }
  }
  __syncthreads();  // the tree's LDS held the counts' lists
  tree_merge128<NW>(acc, nr < NW ? (int)nr : NW, tree);
  // 3. write back
  if (w == 0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int p = h * kWave + l;
      lv[p] = B::from_key(comp_key(acc[h]));
      li[p] = comp_idx(acc[h]);
    }
  }
  for (int e = t; e < a.buf * P; e += kMergeNT) {
    const int r = e / P, b = s_chosen[e % P];
    if (r == 0 && b < 128) continue;  // written above
    lv[(size_t)r * NB + b] = B::fill();
  }
}

static int log2_ceil(int x) {
  int r = 0;
  while ((1 << r) < x) ++r;
  return r;
}

static int bin_buf(int max_m) { return max_m > 1 ? (max_m > (1 << log2_ceil(max_m - 1)) ? max_m : (1 << log2_ceil(max_m - 1))) : max_m; }

// Workspace: candidate lists [rows][kMaxSegLists][128] u64, covered flags,
// per-bin lists (values, indices), per-step pivots and counts, depth_upper,
// and the finish step's per-row / per-block step indices.
constexpr int kMaxSegLists = 32;
static size_t bin_ws(int64_t rows, int num_bins, int buf, int nsteps) {
  size_t b = 0;
  b += (size_t)rows * kMaxSegLists * 128 * 8;  // candidate lists
  b += align_up((size_t)rows * 4, 256);         // covered
  b += (size_t)rows * buf * num_bins * 4;  // lv
  b += (size_t)rows * buf * num_bins * 4;  // li
  b += (size_t)rows * nsteps * 4;          // pivots
  b += (size_t)rows * nsteps * 4;          // counts
  b += 256;                                // depth_upper
  b += 3 * align_up((size_t)rows * 4, 256);  // row_fc, blk_last, row_mlast
  return align_up(b, 256);
}

}  // namespace tx

using namespace tx;

// Path: 0 = candidates where they settle a row, then the full scan for the
// rest (the product path); 1 = the full scan for every row (testing entry
// point only).  Both give the same results.
static int top_dynamic_k_impl(const void* x, int dtype, int64_t rows, int64_t cols, const int32_t* k_rows,
                              int max_k, int block_token, int num_bins, const int32_t* schedule, int num_steps,
                              int guarantee_convergence, int has_replace, double replace_val, void* out_vals, int32_t* out_idx,
                              int32_t* out_valid, int32_t* out_depths, float* out_cutoff, void* workspace,
                              size_t workspace_bytes, hipStream_t stream, int mode);

extern "C" {

size_t tallax_top_dynamic_k_workspace_size(int64_t rows, int num_bins, const int32_t* schedule, int num_steps) {
  if (rows < 0 || num_bins <= 0 || !schedule || num_steps <= 0 || num_steps > kMaxSteps) return 0;
  return bin_ws(rows, num_bins, bin_buf(schedule[num_steps - 1]), num_steps);
}

int tallax_top_dynamic_k(const void* x, int dtype, int64_t rows, int64_t cols, const int32_t* k_rows, int max_k,
                         int block_token, int num_bins, const int32_t* schedule, int num_steps,
                         int guarantee_convergence, int has_replace, double replace_val, void* out_vals,
                         int32_t* out_idx, int32_t* out_valid, int32_t* out_depths, float* out_cutoff,
                         void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return top_dynamic_k_impl(x, dtype, rows, cols, k_rows, max_k, block_token, num_bins, schedule, num_steps,
                            guarantee_convergence, has_replace, replace_val, out_vals, out_idx, out_valid, out_depths, out_cutoff, workspace,
                            workspace_bytes, stream, 0);
}

int tallax_testing_top_dynamic_k_path(const void* x, int dtype, int64_t rows, int64_t cols, const int32_t* k_rows,
                                      int max_k, int block_token, int num_bins, const int32_t* schedule,
                                      int num_steps, int guarantee_convergence, int has_replace,
                                      double replace_val, void* out_vals,
                                      int32_t* out_idx, int32_t* out_valid, int32_t* out_depths, float* out_cutoff,
                                      void* workspace, size_t workspace_bytes, hipStream_t stream, int path) {
  if (path != 0 && path != 1) {
    set_error("path %d is not 0 (candidates) or 1 (scan)", path);
    return kInvalidArgument;
  }
  return top_dynamic_k_impl(x, dtype, rows, cols, k_rows, max_k, block_token, num_bins, schedule, num_steps,
                            guarantee_convergence, has_replace, replace_val, out_vals, out_idx, out_valid, out_depths,
                            out_cutoff, workspace, workspace_bytes, stream, path);
}

}  // extern "C"

static int top_dynamic_k_impl(const void* x, int dtype, int64_t rows, int64_t cols, const int32_t* k_rows,
                              int max_k, int block_token, int num_bins, const int32_t* schedule, int num_steps,
                              int guarantee_convergence, int has_replace, double replace_val, void* out_vals, int32_t* out_idx,
                              int32_t* out_valid, int32_t* out_depths, float* out_cutoff, void* workspace,
                              size_t workspace_bytes, hipStream_t stream, int mode) {
  if (!x || !k_rows || !schedule || !out_vals || !out_idx || !out_valid || !out_depths || !out_cutoff) {
    set_error("null pointer argument");
    return kInvalidArgument;
  }
  if (dtype != kF32 && dtype != kBF16 && dtype != kI32) {
    set_error("dtype %d not supported (f32=0, bf16=1, i32=2)", dtype);
    return kUnsupported;
  }
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
  const int max_m = schedule[num_steps - 1];
  // the bin-packing merge runs for guarantee_convergence unless the last
  // depth is max_k (top_k.py:317-331); the reference derives P from
  // ceil(max_k / (m - 1)) and reads rank 0 of 128 bins
  const bool merge = guarantee_convergence != 0 && max_m != max_k;
  int packed = 0;
  if (merge) {
    if (max_m < 2) {
      set_error("guarantee_convergence needs a last schedule depth >= 2 (or = max_k), got %d", max_m);
      return kInvalidArgument;
    }
    if (num_bins % 128) {
      set_error("guarantee_convergence needs num_bins %% 128 == 0, got %d", num_bins);
      return kUnsupported;
    }
    packed = 1 << log2_ceil((max_k + max_m - 2) / (max_m - 1));
    if (cols + (int64_t)128 * num_bins >= (int64_t)1 << 31) {
      set_error("cols must leave room for the packed columns in int32");
      return kInvalidArgument;
    }
  }
  if (rows == 0) return kOk;
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
  // int32 logits: the replacement is stored into the int32 output, so it is
  // converted toward zero and saturated at the int32 range (NaN -> 0)
  double ri = replace_val != replace_val ? 0.0 : replace_val;
  ri = ri < -2147483648.0 ? -2147483648.0 : (ri > 2147483647.0 ? 2147483647.0 : ri);
  a.replace_i = (int32_t)ri;
  a.merge = merge ? 1 : 0;
  a.num_packed = packed;
  a.out_vals = out_vals; a.out_idx = out_idx; a.out_valid = out_valid; a.out_depths = out_depths;
  a.out_cutoff = out_cutoff;
  char* w = (char*)workspace;
  uint64_t* lists = (uint64_t*)w;
  w += (size_t)rows * kMaxSegLists * 128 * 8;
  int32_t* covered = (int32_t*)w;
  w += align_up((size_t)rows * 4, 256);
  a.lv = (float*)w;
  w += (size_t)rows * buf * num_bins * 4;
  a.li = (int32_t*)w;
  w += (size_t)rows * buf * num_bins * 4;
  a.st_pivot = (float*)w;
  w += (size_t)rows * num_steps * 4;
  a.st_count = (int32_t*)w;
  w += (size_t)rows * num_steps * 4;
  a.upper = (int32_t*)w;
  w += 256;
  a.row_fc = (int32_t*)w;
  w += align_up((size_t)rows * 4, 256);
  a.blk_last = (int32_t*)w;
  w += align_up((size_t)rows * 4, 256);
  a.row_mlast = (int32_t*)w;
  if (rows > 2147483647) { set_error("too many rows"); return kUnsupported; }
  // candidate path: per-segment top-128 lists, then one kernel that settles
  // each row from them (or scans it); otherwise the scan kernel.  The finish
  // step runs inside the select kernel for up to kFinishNT rows, else in its
  // own kernel.
  int nseg = 0, maxv = 0;
  int64_t vps = 0;
  const int min_seg = (num_bins * max_m + 127) / 128;
  // the candidate path starts from the float segment kernel: float inputs only
  const bool cand = mode == 0 && dtype != kI32 && max_m <= kCandRank &&
                    segment_lists_plan(rows, cols, dtype, min_seg < 2 ? 2 : min_seg, &nseg, &maxv, &vps) == kOk &&
                    nseg <= kMaxSegLists;
  const int mc = buf <= 8 ? 8 : 16;
  const size_t lds_scan = (size_t)kBinNT * mc * 8;  // <= 128 KiB
  int st = kOk;
  if (cand) {
    a.lists = lists;
    a.nseg = nseg;
    a.covered = covered;
    st = launch_segment_lists(x, dtype, rows, cols, nseg, maxv, vps, lists, stream);
    if (st) return st;
    const size_t lds_c = cand_lds_bytes(num_bins) > lds_scan ? cand_lds_bytes(num_bins) : lds_scan;
    const hipError_t attr_c8 = set_dynamic_lds_limit((const void*)binned_cand_kernel<8>, 144 * 1024, stream);
    const hipError_t attr_c16 = set_dynamic_lds_limit((const void*)binned_cand_kernel<16>, 144 * 1024, stream);
    if (attr_c8 != hipSuccess || attr_c16 != hipSuccess) { set_error("hipFuncSetAttribute failed"); return kHipError; }
    if (mc == 8)
      hipLaunchKernelGGL(binned_cand_kernel<8>, dim3((unsigned)rows), dim3(kCandNT), lds_c, stream, a);
    else
      hipLaunchKernelGGL(binned_cand_kernel<16>, dim3((unsigned)rows), dim3(kCandNT), lds_c, stream, a);
    st = launch_status("tallax_top_dynamic_k");
    if (st) return st;
    if (rows > kFinishNT) {
      hipLaunchKernelGGL(binned_finish_kernel, dim3(1), dim3(kFinishNT), 0, stream, a);
      st = launch_status("tallax_top_dynamic_k");
      if (st) return st;
    }
  } else {
    const void* kern = dtype == kI32 ? (mc == 8 ? (const void*)binned_lists_kernel<8, int32_t>
                                                : (const void*)binned_lists_kernel<16, int32_t>)
                                     : (mc == 8 ? (const void*)binned_lists_kernel<8, float>
                                                : (const void*)binned_lists_kernel<16, float>);
    if (set_dynamic_lds_limit(kern, 128 * 1024, stream) != hipSuccess) {
      set_error("hipFuncSetAttribute failed");
      return kHipError;
    }
    if (dtype == kI32) {
      if (mc == 8)
        hipLaunchKernelGGL((binned_lists_kernel<8, int32_t>), dim3((unsigned)rows), dim3(kBinNT), lds_scan, stream, a);
      else
        hipLaunchKernelGGL((binned_lists_kernel<16, int32_t>), dim3((unsigned)rows), dim3(kBinNT), lds_scan, stream, a);
    } else {
      if (mc == 8)
        hipLaunchKernelGGL((binned_lists_kernel<8, float>), dim3((unsigned)rows), dim3(kBinNT), lds_scan, stream, a);
      else
        hipLaunchKernelGGL((binned_lists_kernel<16, float>), dim3((unsigned)rows), dim3(kBinNT), lds_scan, stream, a);
    }
    st = launch_status("tallax_top_dynamic_k");
    if (st) return st;
    hipLaunchKernelGGL(binned_finish_kernel, dim3(1), dim3(kFinishNT), 0, stream, a);
    st = launch_status("tallax_top_dynamic_k");
    if (st) return st;
  }
  if (merge) {
    if (cand && rows <= kFinishNT) {  // the finish step was left to the select kernel
      hipLaunchKernelGGL(binned_finish_kernel, dim3(1), dim3(kFinishNT), 0, stream, a);
      st = launch_status("tallax_top_dynamic_k");
      if (st) return st;
    }
    if (dtype == kI32)
      hipLaunchKernelGGL(binned_merge_kernel<int32_t>, dim3((unsigned)rows), dim3(kMergeNT), 0, stream, a);
    else
      hipLaunchKernelGGL(binned_merge_kernel<float>, dim3((unsigned)rows), dim3(kMergeNT), 0, stream, a);
    st = launch_status("tallax_top_dynamic_k");
    if (st) return st;
  }
  if (dtype == kI32)
    hipLaunchKernelGGL((binned_select_kernel<false, int32_t>), dim3((unsigned)rows), dim3(kSelNT), 0, stream, a);
  else if (cand && rows <= kFinishNT && !merge)
    hipLaunchKernelGGL((binned_select_kernel<true, float>), dim3((unsigned)rows), dim3(kSelNT), 0, stream, a);
  else
    hipLaunchKernelGGL((binned_select_kernel<false, float>), dim3((unsigned)rows), dim3(kSelNT), 0, stream, a);
  return launch_status("tallax_top_dynamic_k");
}
