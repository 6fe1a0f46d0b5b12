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

// Pass 1: sorted runs of kWideChunk records, by a stable LSD radix sort on
// the 32-bit key in 8-bit digits (at most four passes; a digit that every key
// of the chunk shares is skipped).  Slot p of the chunk holds record
// (order bits << 32 | tie) of linear index p (column c0 + p, or its reverse
// for descending ties), so the stable sort by key alone is the order of the
// full records; slots past the row hold all-ones records, which stay last.
// The 16384 slots sit record-major inside each wave: slot p = 2048 w + 64 r + l
// is record r (0..31) of lane l of wave w, so a wave's slots in ascending order
// are (r, l).  Per pass:
//   * each wave counts its digits in its own 256 LDS counters (digit-major,
//     NW + 1 words apart) with one atomic per record, r = 0..31 in turn; the
//     atomics of one instruction on one address return in ascending lane order
//     (gfx950; tallax_testing_lds_atomic_order checks it), so the value before
//     a record's increment is its stable rank among the wave's earlier slots
//     of that digit;
//   * an exclusive scan over (digit, wave) in digit-major order gives each
//     pair its start, records move to start + rank through LDS, and the next
//     pass reads them back in slot order.
// (Eight passes of 4-bit digits with per-thread packed counters took 2.93 ms
// at [1024, 201088].)
template <int DT, bool PERM>
__global__ __launch_bounds__(kChunkNT) void sort_chunks_kernel(SortArgs a, int nchunks, uint64_t* out) {
  constexpr int NW = kChunkNT / kWave;
  constexpr int HS = NW + 1;  // counter stride per digit
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
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) {
    kand &= lane_xor(kand, d);
    kor |= lane_xor(kor, d);
  }
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
  const uint32_t varying = kand ^ kor;
#pragma unroll 1
  for (int sh = 0; sh < 32; sh += 8) {
    if (((varying >> sh) & 0xFFu) == 0u) continue;  // every key has this digit: the pass is the identity
#pragma unroll
    for (int d = l; d < 256; d += kWave) hist[d * HS + w] = 0u;  // this wave's counters
    uint32_t rk[kChunkE];
#pragma unroll
    for (int r = 0; r < kChunkE; ++r) {
      const uint32_t d = (uint32_t)(v[r] >> (32 + sh)) & 0xFFu;
      rk[r] = atomicAdd(&hist[d * HS + w], 1u);
    }
    __syncthreads();  // every count is in
    // exclusive scan over i = digit * NW + wave: thread t takes i = 4t .. 4t + 3
    static_assert(256 * NW == 4 * kChunkNT, "four counters per thread in the scan");
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
#pragma unroll
    for (int r = 0; r < kChunkE; ++r) {
      const uint32_t d = (uint32_t)(v[r] >> (32 + sh)) & 0xFFu;
      buf[hist[d * HS + w] + rk[r]] = v[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kChunkE; ++r) v[r] = buf[w * (kChunkE * kWave) + r * kWave + l];
  }
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

}  // namespace tx
