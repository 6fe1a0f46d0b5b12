// Row sort for rows longer than one workgroup's LDS holds (> 16384
// elements): the wide-row route of tax.sort / tumpy.sort / tumpy.argsort.
//
// Reference: sort (tallax/_src/sort.py:768-929) sends such rows to its HBM
// substage engine (sort.py:574-758), a bitonic network whose large-stride
// substages each stream the whole array through HBM.  The results it defines
// are those of a stable sort by (standardised key, tie), S1-S2 in the key
// helpers' terms: ascending or descending key, ties by ascending original
// index (by descending index only on the packed bf16 non-stable descending
// route, utils.py:205-216).
//
// Here every element becomes a 64-bit record (order bits << 32 | tie), where
// the tie is the element's column (or 0x7FFFFFFF - column).  Records are
// unique, so any correct sort of them gives exactly that order, and two
// sorted runs merge without a stability rule.
//   1. sort_chunks_kernel: one 512-thread workgroup sorts each 16384-record
//      chunk of a row in LDS (a stable LSD radix sort on the key, 8-bit
//      digits) and writes the sorted run to the workspace.
//   2. merge_runs_kernel, ceil(log2(chunks)) passes: runs of length L are
//      merged pairwise into runs of 2L, ping-ponging between two workspace
//      buffers.  A workgroup produces 4096 consecutive outputs of one pair:
//      two waves find the tile's start and end on the merge path with a
//      64-way search (one ballot per step, so about three dependent global
//      round trips for a 2^18 run), the tile's inputs are staged in LDS,
//      each thread finds its own 16-output diagonal by binary search in LDS
//      and merges sequentially, and the tile leaves through LDS as coalesced
//      stores.  The last pass writes the permutation, the decoded keys and
//      the gathered second key instead of records.
// Every pass reads and writes each record once (16 bytes per element per
// pass); no kernel waits on another workgroup.
#include <stdint.h>

#include "tallax_hip.h"
#include "tx_block_sort.h"
#include "tx_common.h"
#include "tx_host.h"
#include "tx_scan.h"
#include "tx_sort_keys.h"

namespace tx {

constexpr int kWideChunk = 16384;  // records per chunk sorted in LDS
constexpr int kChunkNT = 512;
constexpr int kChunkE = kWideChunk / kChunkNT;
constexpr int kChunkLds = kWideChunk * 8 + 256 * (kChunkNT / kWave + 1) * 4;  // records + digit counters
constexpr int kMergeNT = 256;
constexpr int kMergeItems = 16;                      // outputs per thread
constexpr int kMergeTile = kMergeNT * kMergeItems;   // outputs per workgroup
constexpr uint32_t kTieMask = 0x7FFFFFFFu;
static_assert((2 * kWideChunk) % kMergeTile == 0, "a merge tile never straddles two pairs of runs");
static_assert(kChunkE * kChunkNT == kWideChunk, "whole chunks per workgroup");

// Stable LSD radix sort by the key (the records' high 32 bits) of the E x NT
// records a workgroup holds in registers in slot order, slot
// (E * 64) w + 64 r + l being record r of lane l of wave w; 8-bit digits, the
// digits in which no key varies skipped.  Slots n and above hold all-ones
// records, which stay last: waves wholly past n neither count nor move theirs.
// buf holds E * NT records, hist 256 * (NT / 64 + 1) counters.  Every thread
// of the workgroup calls it.
//   * each wave counts its digits in its own 256 LDS counters (digit-major,
//     NW + 1 words apart) with one atomic per record, r = 0..E-1 in turn; the
//     atomics of one instruction on one address return in ascending lane order
//     (gfx950; tallax_testing_lds_atomic_order checks it), so the value before
//     a record's increment is its stable rank among the wave's earlier slots
//     of that digit;
//   * an exclusive scan over (digit, wave) in digit-major order gives each
//     pair its start, records move to start + rank through LDS, and the next
//     pass reads them back in slot order.
template <int E, int NT>
__device__ __forceinline__ void radix_sort_slots(uint64_t (&v)[E], uint64_t* buf, uint32_t* hist, uint32_t* wsum,
                                                 uint32_t varying, int n) {
  constexpr int NW = NT / kWave;
  constexpr int HS = NW + 1;  // counter stride per digit
  static_assert(256 * NW == 4 * NT, "four counters per thread in the scan");
  const int t = threadIdx.x, l = lane_id(), w = t / kWave;
  const bool live = w * (E * kWave) < n;  // wave-uniform: the wave holds a slot below n
#pragma unroll 1
  for (int sh = 0; sh < 32; sh += 8) {
    if (((varying >> sh) & 0xFFu) == 0u) continue;  // every key has this digit: the pass is the identity
#pragma unroll
    for (int d = l; d < 256; d += kWave) hist[d * HS + w] = 0u;  // this wave's counters
    uint32_t rk[E];
    if (live) {
#pragma unroll
      for (int r = 0; r < E; ++r) {
        const uint32_t d = (uint32_t)(v[r] >> (32 + sh)) & 0xFFu;
        rk[r] = atomicAdd(&hist[d * HS + w], 1u);
      }
    }
    __syncthreads();  // every count is in
    // exclusive scan over i = digit * NW + wave: thread t takes i = 4t .. 4t + 3
    const int d0 = (4 * t) / NW, w0 = (4 * t) % NW;
    uint32_t cq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) cq[q] = hist[d0 * HS + w0 + q];
    const uint32_t run = cq[0] + cq[1] + cq[2] + cq[3];
    const uint32_t incl = wave_incl_scan(run);
    if (l == kWave - 1) wsum[w] = incl;
    __syncthreads();
    uint32_t pre = incl - run;
#pragma unroll
    for (int i = 0; i < NW; ++i) pre += i < w ? wsum[i] : 0u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      hist[d0 * HS + w0 + q] = pre;
      pre += cq[q];
    }
    __syncthreads();
    if (live) {
#pragma unroll
      for (int r = 0; r < E; ++r) {
        const uint32_t d = (uint32_t)(v[r] >> (32 + sh)) & 0xFFu;
        buf[hist[d * HS + w] + rk[r]] = v[r];
      }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < E; ++r) {
      const int L = w * (E * kWave) + r * kWave + l;
      v[r] = L < n ? buf[L] : ~0ull;
    }
  }
}

// Pass 1: sorted runs of kWideChunk records, by a stable LSD radix sort on
// the 32-bit key in 8-bit digits (radix_sort_slots: at most four passes; a
// digit that every key of the chunk shares is skipped).  Slot p of the chunk
// holds record (order bits << 32 | tie) of linear index p (column c0 + p, or
// its reverse for descending ties), so the stable sort by key alone is the
// order of the full records; slots past the row hold all-ones records, which
// stay last.  (Eight passes of 4-bit digits with per-thread packed counters
// took 2.93 ms at [1024, 201088]; these four, 1.60 ms.)
template <int DT, bool PERM>
__global__ __launch_bounds__(kChunkNT) void sort_chunks_kernel(SortArgs a, int nchunks, uint64_t* out) {
  constexpr int NW = kChunkNT / kWave;
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* buf = (uint64_t*)smem;                     // kWideChunk records
  uint32_t* hist = (uint32_t*)(buf + kWideChunk);      // 256 * HS counters
  __shared__ uint32_t wsum[NW];
  __shared__ uint32_t red[2][NW];
  const int t = threadIdx.x, l = lane_id(), w = t / kWave;
  const int64_t row = blockIdx.x / (unsigned)nchunks;
  const int c = (int)(blockIdx.x - row * nchunks);
  const int64_t base = row * a.cols;
  const int64_t c0 = (int64_t)c * kWideChunk;
  const int n = (int)min((int64_t)kWideChunk, a.cols - c0);
  // records in slot order (coalesced reads, every load of the chunk in
  // flight at once), and which key bits vary
  uint32_t kand = ~0u, kor = 0u;
  uint64_t v[kChunkE];
  {
    uint32_t raw[kChunkE];
    int32_t src[kChunkE];
#pragma unroll
    for (int r = 0; r < kChunkE; ++r) {
      const int L = w * (kChunkE * kWave) + r * kWave + l;
      src[r] = (int32_t)(c0 + (a.ties_desc ? n - 1 - L : L));
      if (PERM && L < n) src[r] = a.perm_in[base + src[r]];
    }
#pragma unroll
    for (int r = 0; r < kChunkE; ++r) {
      const int L = w * (kChunkE * kWave) + r * kWave + l;
      raw[r] = L < n ? key_bits_at<DT>(a.key, base + src[r]) : 0u;
    }
#pragma unroll
    for (int r = 0; r < kChunkE; ++r) {
      const int L = w * (kChunkE * kWave) + r * kWave + l;
      v[r] = ~0ull;
      if (L < n) {
        uint32_t k = order_from_bits(raw[r], DT);
        if (a.descending) k = ~k;
        const uint32_t p = (uint32_t)(c0 + (a.ties_desc ? n - 1 - L : L));
        const uint32_t tie = a.ties_desc ? kTieMask - p : p;
        v[r] = ((uint64_t)k << 32) | tie;
        kand &= k;
        kor |= k;
      }
    }
  }
  kand = wave_and_u32(kand);
  kor = wave_or_u32(kor);
  if (l == 0) {
    red[0][w] = kand;
    red[1][w] = kor;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    kand &= red[0][i];
    kor |= red[1][i];
  }
  // bfloat16 keys: the low 16 order bits follow from the high 16 (as in
  // sort_row_radix_kernel), so only the high digits are sorted
  const uint32_t varying = (kand ^ kor) & (DT == kBF16 ? 0xFFFF0000u : ~0u);
  radix_sort_slots<kChunkE, kChunkNT>(v, buf, hist, wsum, varying, n);
  uint64_t* dst = out + base + c0;
#pragma unroll
  for (int r = 0; r < kChunkE; ++r) {
    const int L = w * (kChunkE * kWave) + r * kWave + l;
    if (L < n) dst[L] = v[r];
  }
}

// Merge path: the number of A records among the first d records of the
// merge of sorted A[0, la) and B[0, lb), i.e. the first i in
// [max(0, d - lb), min(d, la)) with A[i] > B[d - 1 - i], or min(d, la) when
// there is none.  One wave; every lane returns the same value.  Each step
// probes 64 positions (at most n / 64 apart) and keeps the interval between
// the last false and the first true probe.
__device__ int merge_split_wave(const uint64_t* A, int la, const uint64_t* B, int lb, int d) {
  const int l = lane_id();
  int lo = max(0, d - lb), hi = min(d, la);
  while (hi > lo) {
    const int n = hi - lo;
    const bool small = n <= kWave;
    const int q = small ? lo + l : lo + (int)(((int64_t)(l + 1) * n) / kWave) - 1;
    const bool f = (!small || l < n) && A[q] > B[d - 1 - q];
    const uint64_t b = __ballot(f);
    if (!b) return hi;
    const int l0 = __ffsll((unsigned long long)b) - 1;
    if (small) return lo + l0;
    const int qprev = lo + (int)(((int64_t)l0 * n) / kWave) - 1;  // lo - 1 for l0 = 0
    hi = lo + (int)(((int64_t)(l0 + 1) * n) / kWave) - 1;         // a true probe
    lo = qprev + 1;
  }
  return lo;
}

// One merge pass over runs of length `run`: the pair of runs starting at
// column s = 2 run j merges into columns [s, s + 2 run) of dst.  A run with
// no partner (the row's last) is copied.  FINAL writes the outputs instead.
// LDS slot of merge-tile record j: one spare slot per 16 records, so that
// the 64 lanes of a wave, each merging its own run of 16 outputs (records 16
// apart), spread over the banks instead of all hitting one.
__device__ __forceinline__ int ms(int j) { return j + (j >> 4); }

template <bool FINAL>
__global__ __launch_bounds__(kMergeNT) void merge_runs_kernel(SortArgs a, const uint64_t* src, uint64_t* dst,
                                                              int64_t run, int tiles) {
  __shared__ uint64_t lds[kMergeTile + kMergeTile / 16];  // record j at ms(j)
  __shared__ int split[2];
  const int t = threadIdx.x, w = t / kWave;
  // Workgroups go to the 8 XCDs round-robin, each with its own L2: the tile
  // order is remapped so that every XCD takes a contiguous range of tiles, and
  // neighbouring tiles, whose merge-path searches probe the same lines of the
  // same runs, share an L2.
  const unsigned nwg = gridDim.x;
  const unsigned vb = nwg % 8u == 0u ? (blockIdx.x % 8u) * (nwg / 8u) + blockIdx.x / 8u : blockIdx.x;
  const int64_t row = vb / (unsigned)tiles;
  const int ti = (int)(vb - row * tiles);
  const int64_t base = row * a.cols;
  const int64_t o0 = (int64_t)ti * kMergeTile;  // first output column of the tile
  const int64_t s = o0 / (2 * run) * (2 * run);
  const int la = (int)min(run, a.cols - s);
  const int lb = (int)max((int64_t)0, min(run, a.cols - s - run));
  const int d0 = (int)(o0 - s);
  const int count = min(kMergeTile, la + lb - d0);
  const uint64_t* A = src + base + s;
  const uint64_t* B = A + run;  // read only where lb > 0
  if (w < 2) {
    const int sp = merge_split_wave(A, la, B, lb, d0 + w * count);
    if (lane_id() == 0) split[w] = sp;
  }
  __syncthreads();
  const int a0 = split[0];
  const int na = split[1] - a0;
  const int b0 = d0 - a0;
  const int nb = count - na;
  {
    uint64_t st[kMergeItems];  // every load of the tile in flight at once
#pragma unroll
    for (int k = 0; k < kMergeItems; ++k) {
      const int j = k * kMergeNT + t;
      st[k] = j < count ? (j < na ? A[a0 + j] : B[b0 + (j - na)]) : 0ull;
    }
#pragma unroll
    for (int k = 0; k < kMergeItems; ++k) {
      const int j = k * kMergeNT + t;
      if (j < count) lds[ms(j)] = st[k];
    }
  }
  __syncthreads();
  uint64_t out[kMergeItems];
  const int dt = t * kMergeItems;
  if (dt < count) {
    int lo = max(0, dt - nb), hi = min(dt, na);
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (lds[ms(mid)] > lds[ms(na + dt - 1 - mid)]) hi = mid;
      else lo = mid + 1;
    }
    int ia = lo, ib = dt - lo;
    uint64_t x = ia < na ? lds[ms(ia)] : ~0ull;
    uint64_t y = ib < nb ? lds[ms(na + ib)] : ~0ull;
#pragma unroll
    for (int r = 0; r < kMergeItems; ++r) {
      const bool take_a = x < y;
      out[r] = take_a ? x : y;
      if (take_a) {
        ++ia;
        x = ia < na ? lds[ms(ia)] : ~0ull;
      } else {
        ++ib;
        y = ib < nb ? lds[ms(na + ib)] : ~0ull;
      }
    }
  }
  __syncthreads();
  if (dt < count) {
#pragma unroll
    for (int r = 0; r < kMergeItems; ++r)
      if (dt + r < count) lds[ms(dt + r)] = out[r];
  }
  __syncthreads();
  if (!FINAL) {
    for (int j = t; j < count; j += kMergeNT) dst[base + o0 + j] = lds[ms(j)];
    return;
  }
  // outputs: source columns, then the gathered second key, each batch of
  // dependent loads in flight at once
  int32_t col[kMergeItems];  // columns are < 2^31
#pragma unroll
  for (int k = 0; k < kMergeItems; ++k) {
    const int j = k * kMergeNT + t;
    col[k] = 0;
    if (j < count) {
      const uint32_t tie = (uint32_t)lds[ms(j)];
      const int32_t pos = (int32_t)(a.ties_desc ? kTieMask - tie : tie);
      col[k] = a.perm_in ? a.perm_in[base + pos] : pos;
    }
  }
#pragma unroll
  for (int k = 0; k < kMergeItems; ++k) {
    const int j = k * kMergeNT + t;
    if (j >= count) continue;
    a.perm_out[base + o0 + j] = col[k];
    if (a.key_out) {
      uint32_t key = (uint32_t)(lds[ms(j)] >> 32);
      if (a.descending) key = ~key;
      store_sorted(a.key_out, a.key_out_dtype, a.key_dtype, base + o0 + j, key);
    }
  }
  if (a.aux_out) {
    uint32_t u[kMergeItems];
    if (a.aux_dtype == kBF16) {
#pragma unroll
      for (int k = 0; k < kMergeItems; ++k)
        u[k] = k * kMergeNT + t < count ? key_bits_at<kBF16>(a.aux, base + col[k]) : 0u;
    } else {
#pragma unroll
      for (int k = 0; k < kMergeItems; ++k)
        u[k] = k * kMergeNT + t < count ? key_bits_at<kF32>(a.aux, base + col[k]) : 0u;
    }
#pragma unroll
    for (int k = 0; k < kMergeItems; ++k) {
      const int j = k * kMergeNT + t;
      if (j < count)
        store_sorted(a.aux_out, a.aux_out_dtype, a.aux_dtype, base + o0 + j, order_from_bits(u[k], a.aux_dtype));
    }
  }
}

// ---------------------------------------------------------------------------
// Multiway merge by splitters (rows of 3 to kBucketMaxRuns chunks): one pass
// instead of ceil(log2 chunks) pairwise merge passes.
//   * bucket_split_kernel, one workgroup per row: every kBucketStride-th record
//     of every sorted run is a sample (record (a + 1) G - 1 of a run, G the
//     stride); the samples (at most 4096) are sorted by a block bitonic
//     network, and every m-th one of them in that order is a splitter s_k.
//     For every splitter and run, the run's first position p_kj with a record
//     >= s_k: the run's samples below s_k, c, put it in [c G, (c + 1) G), so a
//     binary search of G records finds it.  Bucket k holds the records in
//     [s_k, s_k+1).  From run j it takes at most (q_j + 1) G records, q_j its
//     samples in the bucket, and the bucket's samples number at most m, so a
//     bucket never exceeds (m + runs) G records: m is chosen so that this is
//     the bucket kernel's capacity.  The table holds every p_kj and each
//     bucket's first output rank, sum_j p_kj.
//   * bucket_sort_kernel, one workgroup per (row, bucket): the bucket's part of
//     every run is loaded, run after run in tie order (chunk j holds columns
//     [j, j + 1) kWideChunk: ascending ties take the runs in order, descending
//     ones in reverse).  Inside one run the records are sorted, and between
//     runs records of equal keys then come in tie order.  So the stable radix sort by the key
//     alone (radix_sort_slots) gives the records' order, and the outputs
//     (permutation, keys, gathered second key) are written at the bucket's
//     first output rank.
// Traffic: the chunk pass (4 bytes in, 8 out per element), then 8 in and the
// outputs out: 28 bytes per element with keys and indices out, against 76 for
// four pairwise merge passes at [1024, 201088].
// ---------------------------------------------------------------------------
constexpr int kBucketStride = 256;       // G: records between samples
constexpr int kBucketMaxRuns = 56;       // (m >= 8) + runs <= 64: buckets of at most 64 G = 16384 records
constexpr int kSplitNT = 1024;
constexpr int kSplitSamples = 4096;      // >= kBucketMaxRuns * kWideChunk / kBucketStride
constexpr int kBucketNT = 512;
static_assert(kBucketMaxRuns * (kWideChunk / kBucketStride) <= kSplitSamples, "every sample fits the sort");

struct BucketPlan {
  int runs;     // chunks of a row
  int samples;  // S: samples of a row
  int m;        // samples per bucket
  int K;        // buckets of a row
  int E;        // records per thread of the bucket kernel (capacity E * kBucketNT)
};

__host__ __device__ inline int run_len(int64_t cols, int j) {
  const int64_t left = cols - (int64_t)j * kWideChunk;
  return (int)(left < kWideChunk ? left : kWideChunk);
}

__global__ __launch_bounds__(kSplitNT) void bucket_split_kernel(SortArgs a, BucketPlan bp, const uint64_t* runs,
                                                                int32_t* table) {
  __shared__ uint64_t srt[kSplitSamples];   // samples, sorted
  __shared__ uint64_t per[kSplitSamples];   // samples in run order (each run's ascending)
  __shared__ int sp[kBucketMaxRuns + 1];    // first sample of each run
  __shared__ int soff[kSplitSamples / 8 + 2];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t base = row * a.cols;
  const int R = bp.runs, G = kBucketStride;
  if (t == 0) {
    int acc = 0;
    for (int j = 0; j < R; ++j) {
      sp[j] = acc;
      acc += run_len(a.cols, j) / G;
    }
    sp[R] = acc;
  }
  for (int k = t; k <= bp.K; k += kSplitNT) soff[k] = 0;
  __syncthreads();
  // sample i = 4t + r: run j with sp[j] <= i < sp[j + 1], record (i - sp[j] + 1) G - 1 of it
  uint64_t v[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = 4 * t + r;
    v[r] = ~0ull;
    if (i < bp.samples) {
      int j = 0;
      while (sp[j + 1] <= i) ++j;
      v[r] = runs[base + (int64_t)j * kWideChunk + (int64_t)(i - sp[j] + 1) * G - 1];
      per[i] = v[r];
    }
  }
  block_bitonic_sort_c<uint64_t, 4, kSplitSamples, false>(v, srt);
#pragma unroll
  for (int r = 0; r < 4; ++r) srt[4 * t + r] = v[r];
  __syncthreads();
  // p_kj for k = 0..K (k = 0: 0; k = K: the run's length), one (k, j) per thread in turn
  int32_t* tp = table + row * (int64_t)(bp.K + 1) * (R + 1);  // [(K + 1) R] positions, then [K + 1] offsets
  for (int q = t; q < (bp.K + 1) * R; q += kSplitNT) {
    const int k = q / R, j = q - k * R;
    const int len = run_len(a.cols, j);
    int pos;
    if (k == 0) {
      pos = 0;
    } else if (k == bp.K) {
      pos = len;
    } else {
      const uint64_t sk = srt[k * bp.m];
      // samples of run j below sk (each run's samples ascend)
      int lo = sp[j], hi = sp[j + 1];
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (per[mid] < sk) lo = mid + 1;
        else hi = mid;
      }
      const int c = lo - sp[j];
      // first record >= sk in [c G, min((c + 1) G - 1, len)]
      int l0 = c * G, h0 = c < sp[j + 1] - sp[j] ? (c + 1) * G - 1 : len;
      const uint64_t* rj = runs + base + (int64_t)j * kWideChunk;
      while (l0 < h0) {
        const int mid = (l0 + h0) >> 1;
        if (rj[mid] < sk) l0 = mid + 1;
        else h0 = mid;
      }
      pos = l0;
    }
    tp[q] = pos;
    atomicAdd(&soff[k], pos);
  }
  __syncthreads();
  for (int k = t; k <= bp.K; k += kSplitNT) tp[(bp.K + 1) * R + k] = soff[k];
}

template <int E>
__global__ __launch_bounds__(kBucketNT) void bucket_sort_kernel(SortArgs a, BucketPlan bp, const uint64_t* runs,
                                                                const int32_t* table) {
  constexpr int NW = kBucketNT / kWave;
  constexpr int CAP = E * kBucketNT;
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* buf = (uint64_t*)smem;                 // CAP records
  uint32_t* hist = (uint32_t*)(buf + CAP);         // 256 * (NW + 1) counters
  __shared__ uint32_t wsum[NW];
  __shared__ uint32_t red[2][NW];
  __shared__ int s_lo[kBucketMaxRuns], s_off[kBucketMaxRuns + 1];
  const int t = threadIdx.x, l = lane_id(), w = t / kWave;
  const int R = bp.runs;
  const int64_t row = blockIdx.x / (unsigned)bp.K;
  const int k = (int)(blockIdx.x - row * bp.K);
  const int64_t base = row * a.cols;
  const int32_t* tp = table + row * (int64_t)(bp.K + 1) * (R + 1);
  if (w == 0) {  // the bucket's range in each run and its slots, by a wave scan
    // runs in tie order: chunk j holds columns [j, j + 1) * kWideChunk, so
    // with descending ties (tie = kTieMask - column) the last run comes first
    int lo = 0, sz = 0;
    if (l < R) {
      const int j = a.ties_desc ? R - 1 - l : l;
      lo = tp[k * R + j];
      sz = tp[(k + 1) * R + j] - lo;
    }
    int tot;
    const int pre = wave_exscan_i32(sz, tot);
    if (l < R) {
      s_lo[l] = lo;
      s_off[l] = pre;
    }
    if (l == 0) s_off[R] = tot;
  }
  __syncthreads();
  const int n = s_off[R];  // at most CAP (the split's bound)
  if (n > CAP) return;     // never taken; keeps a broken table from writing past the LDS buffer
  const int64_t o0 = tp[(bp.K + 1) * R + k];
  // slot L is record L - s_off[i] of the bucket's part of the i-th run (in tie
  // order); the slots of a thread ascend, so its run index only moves up
  uint32_t kand = ~0u, kor = 0u;
  uint64_t v[E];
  {
    const uint64_t* src[E];
    int i = 0;
#pragma unroll
    for (int r = 0; r < E; ++r) {
      const int L = w * (E * kWave) + r * kWave + l;
      src[r] = nullptr;
      if (L < n) {
        while (s_off[i + 1] <= L) ++i;
        const int j = a.ties_desc ? R - 1 - i : i;
        src[r] = runs + base + (int64_t)j * kWideChunk + s_lo[i] + (L - s_off[i]);
      }
    }
#pragma unroll
    for (int r = 0; r < E; ++r) v[r] = src[r] ? *src[r] : ~0ull;
#pragma unroll
    for (int r = 0; r < E; ++r) {
      if (src[r]) {
        kand &= (uint32_t)(v[r] >> 32);
        kor |= (uint32_t)(v[r] >> 32);
      }
    }
  }
  kand = wave_and_u32(kand);
  kor = wave_or_u32(kor);
  if (l == 0) {
    red[0][w] = kand;
    red[1][w] = kor;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    kand &= red[0][i];
    kor |= red[1][i];
  }
  radix_sort_slots<E, kBucketNT>(v, buf, hist, wsum, (kand ^ kor) & (a.key_dtype == kBF16 ? 0xFFFF0000u : ~0u), n);
  // outputs at ranks o0 + slot: the source column, then the sorted key and
  // the gathered second key, each batch of dependent loads in flight at once
  int32_t col[E];
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int L = w * (E * kWave) + r * kWave + l;
    col[r] = 0;
    if (L < n) {
      const uint32_t tie = (uint32_t)v[r];
      const int32_t pos = (int32_t)(a.ties_desc ? kTieMask - tie : tie);
      col[r] = a.perm_in ? a.perm_in[base + pos] : pos;
    }
  }
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int L = w * (E * kWave) + r * kWave + l;
    if (L >= n) continue;
    a.perm_out[base + o0 + L] = col[r];
    if (a.key_out) {
      uint32_t key = (uint32_t)(v[r] >> 32);
      if (a.descending) key = ~key;
      store_sorted(a.key_out, a.key_out_dtype, a.key_dtype, base + o0 + L, key);
    }
  }
  if (a.aux_out) {
    uint32_t u[E];
    if (a.aux_dtype == kBF16) {
#pragma unroll
      for (int r = 0; r < E; ++r)
        u[r] = w * (E * kWave) + r * kWave + l < n ? key_bits_at<kBF16>(a.aux, base + col[r]) : 0u;
    } else {
#pragma unroll
      for (int r = 0; r < E; ++r)
        u[r] = w * (E * kWave) + r * kWave + l < n ? key_bits_at<kF32>(a.aux, base + col[r]) : 0u;
    }
#pragma unroll
    for (int r = 0; r < E; ++r) {
      const int L = w * (E * kWave) + r * kWave + l;
      if (L < n)
        store_sorted(a.aux_out, a.aux_out_dtype, a.aux_dtype, base + o0 + L, order_from_bits(u[r], a.aux_dtype));
    }
  }
}

// Rows of at most E * kChunkNT (<= kWideChunk) elements sorted whole by one
// workgroup: the chunk pass's records and radix sort, then the outputs
// straight from the sorted records (the bucket pass's output step at rank 0).
// An LDS bitonic network moves O(n log^2 n) records per row; this sort moves
// each record once per varying digit ([256, 16384] f32: 32.4 us against
// 190.8 us for the network).  For bfloat16 keys the low 16 order bits follow
// from the high 16 (they are zero or the sign's complement, and every NaN
// has one order), so only the high two digits are sorted.
template <int DT, bool PERM, int E>
__global__ __launch_bounds__(kChunkNT) void sort_row_radix_kernel(SortArgs a) {
  constexpr int NW = kChunkNT / kWave;
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* buf = (uint64_t*)smem;                 // E * kChunkNT records
  uint32_t* hist = (uint32_t*)(buf + E * kChunkNT);  // 256 * (NW + 1) counters
  __shared__ uint32_t wsum[NW];
  __shared__ uint32_t red[2][NW];
  const int t = threadIdx.x, l = lane_id(), w = t / kWave;
  const int64_t row = blockIdx.x;
  const int64_t base = row * a.cols;
  const int n = (int)a.cols;  // 1 <= n <= E * kChunkNT (host routing)
  uint32_t kand = ~0u, kor = 0u;
  uint64_t v[E];
  {
    uint32_t raw[E];
    int32_t src[E];
#pragma unroll
    for (int r = 0; r < E; ++r) {
      const int L = w * (E * kWave) + r * kWave + l;
      src[r] = a.ties_desc ? n - 1 - L : L;
      if (PERM && L < n) src[r] = a.perm_in[base + src[r]];
    }
#pragma unroll
    for (int r = 0; r < E; ++r) {
      const int L = w * (E * kWave) + r * kWave + l;
      raw[r] = L < n ? key_bits_at<DT>(a.key, base + src[r]) : 0u;
    }
#pragma unroll
    for (int r = 0; r < E; ++r) {
      const int L = w * (E * kWave) + r * kWave + l;
      v[r] = ~0ull;
      if (L < n) {
        uint32_t k = order_from_bits(raw[r], DT);
        if (a.descending) k = ~k;
        const uint32_t p = (uint32_t)(a.ties_desc ? n - 1 - L : L);
        const uint32_t tie = a.ties_desc ? kTieMask - p : p;
        v[r] = ((uint64_t)k << 32) | tie;
        kand &= k;
        kor |= k;
      }
    }
  }
  kand = wave_and_u32(kand);
  kor = wave_or_u32(kor);
  if (l == 0) {
    red[0][w] = kand;
    red[1][w] = kor;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    kand &= red[0][i];
    kor |= red[1][i];
  }
  const uint32_t varying = (kand ^ kor) & (DT == kBF16 ? 0xFFFF0000u : ~0u);
  radix_sort_slots<E, kChunkNT>(v, buf, hist, wsum, varying, n);
  int32_t col[E];
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int L = w * (E * kWave) + r * kWave + l;
    col[r] = 0;
    if (L < n) {
      const uint32_t tie = (uint32_t)v[r];
      const int32_t pos = (int32_t)(a.ties_desc ? kTieMask - tie : tie);
      col[r] = PERM ? a.perm_in[base + pos] : pos;
    }
  }
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int L = w * (E * kWave) + r * kWave + l;
    if (L >= n) continue;
    a.perm_out[base + L] = col[r];
    if (a.key_out) {
      uint32_t key = (uint32_t)(v[r] >> 32);
      if (a.descending) key = ~key;
      store_sorted(a.key_out, a.key_out_dtype, a.key_dtype, base + L, key);
    }
  }
  if (a.aux_out) {
    uint32_t u[E];
    if (a.aux_dtype == kBF16) {
#pragma unroll
      for (int r = 0; r < E; ++r)
        u[r] = w * (E * kWave) + r * kWave + l < n ? key_bits_at<kBF16>(a.aux, base + col[r]) : 0u;
    } else {
#pragma unroll
      for (int r = 0; r < E; ++r)
        u[r] = w * (E * kWave) + r * kWave + l < n ? key_bits_at<kF32>(a.aux, base + col[r]) : 0u;
    }
#pragma unroll
    for (int r = 0; r < E; ++r) {
      const int L = w * (E * kWave) + r * kWave + l;
      if (L < n)
        store_sorted(a.aux_out, a.aux_out_dtype, a.aux_dtype, base + L, order_from_bits(u[r], a.aux_dtype));
    }
  }
}

template <int DT, bool PERM, int E>
static int launch_row_radix_e(const SortArgs& a, int64_t rows, hipStream_t s) {
  const int lds = E * kChunkNT * 8 + 256 * (kChunkNT / kWave + 1) * 4;
  const hipError_t attr = set_dynamic_lds_limit((const void*)sort_row_radix_kernel<DT, PERM, E>, lds, s);
  if (attr != hipSuccess) {
    set_error("hipFuncSetAttribute: %s", hipGetErrorString(attr));
    return kHipError;
  }
  hipLaunchKernelGGL((sort_row_radix_kernel<DT, PERM, E>), dim3((unsigned)rows), dim3(kChunkNT), lds, s, a);
  return kOk;
}

template <int DT, bool PERM>
static int launch_row_radix_dt(const SortArgs& a, int64_t rows, hipStream_t s) {
  if (a.cols <= 4 * kChunkNT) return launch_row_radix_e<DT, PERM, 4>(a, rows, s);
  if (a.cols <= 8 * kChunkNT) return launch_row_radix_e<DT, PERM, 8>(a, rows, s);
  if (a.cols <= 16 * kChunkNT) return launch_row_radix_e<DT, PERM, 16>(a, rows, s);
  return launch_row_radix_e<DT, PERM, 32>(a, rows, s);
}

template <int DT, bool PERM>
static int launch_chunks(const SortArgs& a, int64_t rows, int64_t nchunks, uint64_t* out, hipStream_t s) {
  const hipError_t attr = set_dynamic_lds_limit((const void*)sort_chunks_kernel<DT, PERM>, kChunkLds, s);
  if (attr != hipSuccess) {
    set_error("hipFuncSetAttribute: %s", hipGetErrorString(attr));
    return kHipError;
  }
  hipLaunchKernelGGL((sort_chunks_kernel<DT, PERM>), dim3((unsigned)(rows * nchunks)), dim3(kChunkNT), kChunkLds, s,
                     a, (int)nchunks, out);
  return kOk;
}

static int wide_passes(int64_t cols) {
  const int64_t nchunks = (cols + kWideChunk - 1) / kWideChunk;
  int passes = 0;
  while (((int64_t)1 << passes) < nchunks) ++passes;
  return passes;
}

size_t sort_wide_workspace_bytes(int64_t rows, int64_t cols) {
  if (cols <= kWideChunk || rows <= 0) return 0;
  return (size_t)(wide_passes(cols) > 1 ? 2 : 1) * (size_t)rows * (size_t)cols * sizeof(uint64_t);
}

int launch_sort_wide(const SortArgs& a, int64_t rows, void* ws, size_t ws_bytes, hipStream_t s) {
  const int64_t cols = a.cols;
  if (cols > (int64_t)kTieMask) {
    set_error("rows of %lld elements exceed the wide sort's limit of 2^31 - 1", (long long)cols);
    return kUnsupported;
  }
  const int64_t nchunks = (cols + kWideChunk - 1) / kWideChunk;
  const int64_t tiles = (cols + kMergeTile - 1) / kMergeTile;
  if (rows * tiles > 2147483647 || rows * nchunks > 2147483647) {
    set_error("sort of %lld x %lld elements needs more than 2^31 - 1 workgroups", (long long)rows, (long long)cols);
    return kUnsupported;
  }
  const size_t need = sort_wide_workspace_bytes(rows, cols);
  if (!ws || ws_bytes < need) {
    set_error("rows of %lld elements need a workspace of %zu bytes, got %zu", (long long)cols, need,
              ws ? ws_bytes : (size_t)0);
    return kWorkspaceTooSmall;
  }
  uint64_t* buf[2] = {(uint64_t*)ws, (uint64_t*)ws + (size_t)rows * (size_t)cols};
  int st = a.key_dtype == kBF16 ? (a.perm_in ? launch_chunks<kBF16, true>(a, rows, nchunks, buf[0], s)
                                              : launch_chunks<kBF16, false>(a, rows, nchunks, buf[0], s))
         : a.key_dtype == kI32  ? (a.perm_in ? launch_chunks<kI32, true>(a, rows, nchunks, buf[0], s)
                                              : launch_chunks<kI32, false>(a, rows, nchunks, buf[0], s))
                                : (a.perm_in ? launch_chunks<kF32, true>(a, rows, nchunks, buf[0], s)
                                              : launch_chunks<kF32, false>(a, rows, nchunks, buf[0], s));
  if (!st) st = launch_status("tallax_sort_rows (chunks)");
  if (st) return st;
  // rows of 3 .. kBucketMaxRuns chunks: the multiway merge by splitters
  // (the table lives in the second workspace buffer, which exists whenever
  // there are two or more pairwise passes)
  if (nchunks >= 3 && nchunks <= kBucketMaxRuns) {
    BucketPlan bp;
    bp.runs = (int)nchunks;
    bp.samples = 0;
    for (int j = 0; j < bp.runs; ++j) bp.samples += run_len(cols, j) / kBucketStride;
    bp.E = bp.runs <= 24 ? 16 : 32;                    // capacity 8192 or 16384 records
    bp.m = (bp.E * kBucketNT) / kBucketStride - bp.runs;  // (m + runs) G = capacity
    bp.K = (bp.samples + bp.m - 1) / bp.m;
    if (bp.K < 1) bp.K = 1;
    if (rows * bp.K > 2147483647) {
      set_error("sort of %lld rows needs more than 2^31 - 1 workgroups", (long long)rows);
      return kUnsupported;
    }
    int32_t* table = (int32_t*)buf[1];
    hipLaunchKernelGGL(bucket_split_kernel, dim3((unsigned)rows), dim3(kSplitNT), 0, s, a, bp, buf[0], table);
    st = launch_status("tallax_sort_rows (splitters)");
    if (st) return st;
    const int lds = bp.E * kBucketNT * 8 + 256 * (kBucketNT / kWave + 1) * 4;
    const void* kfn = bp.E == 16 ? (const void*)bucket_sort_kernel<16> : (const void*)bucket_sort_kernel<32>;
    const hipError_t attr = set_dynamic_lds_limit(kfn, lds, s);
    if (attr != hipSuccess) {
      set_error("hipFuncSetAttribute: %s", hipGetErrorString(attr));
      return kHipError;
    }
    const dim3 grid((unsigned)(rows * bp.K));
    if (bp.E == 16)
      hipLaunchKernelGGL(bucket_sort_kernel<16>, grid, dim3(kBucketNT), lds, s, a, bp, (const uint64_t*)buf[0], table);
    else
      hipLaunchKernelGGL(bucket_sort_kernel<32>, grid, dim3(kBucketNT), lds, s, a, bp, (const uint64_t*)buf[0], table);
    return launch_status("tallax_sort_rows (buckets)");
  }
  const int passes = wide_passes(cols);
  for (int p = 0; p < passes && !st; ++p) {
    const int64_t run = (int64_t)kWideChunk << p;
    const dim3 grid((unsigned)(rows * tiles));
    if (p + 1 == passes)
      hipLaunchKernelGGL(merge_runs_kernel<true>, grid, dim3(kMergeNT), 0, s, a, buf[p & 1], nullptr, run,
                         (int)tiles);
    else
      hipLaunchKernelGGL(merge_runs_kernel<false>, grid, dim3(kMergeNT), 0, s, a, buf[p & 1], buf[(p + 1) & 1],
                         run, (int)tiles);
    st = launch_status("tallax_sort_rows (merge)");
  }
  return st;
}

int launch_sort_row_radix(const SortArgs& a, int64_t rows, hipStream_t s) {
  if (a.cols < 1 || a.cols > kWideChunk) {
    set_error("row radix sort: %lld columns outside [1, %d]", (long long)a.cols, kWideChunk);
    return kInvalidArgument;
  }
  if (a.key_dtype == kBF16)
    return a.perm_in ? launch_row_radix_dt<kBF16, true>(a, rows, s) : launch_row_radix_dt<kBF16, false>(a, rows, s);
  if (a.key_dtype == kI32)
    return a.perm_in ? launch_row_radix_dt<kI32, true>(a, rows, s) : launch_row_radix_dt<kI32, false>(a, rows, s);
  return a.perm_in ? launch_row_radix_dt<kF32, true>(a, rows, s) : launch_row_radix_dt<kF32, false>(a, rows, s);
}

}  // namespace tx
