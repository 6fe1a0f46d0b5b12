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
//   Kernel A, seg_select_kernel: one workgroup per (segment, row).  A row is
//   either one segment of a 512-thread workgroup (up to 32 16-byte vectors per
//   thread, no second kernel) or `nseg` segments of 256 threads, sized so that
//   ~4 workgroups run per CU.  Every load of the segment is issued up front
//   into registers, then:
//     - each thread takes the maximum of its elements as a monotone key
//       (integer max over raw bits, packed for bf16 pairs);
//     - a lower bound L on the segment's k-th key: each wave sorts its 64
//       per-thread maxima (wave64 bitonic network) and L is the minimum over
//       the waves of their ceil(k/waves)-th largest maximum, so at least k
//       elements are >= L;
//     - vectors whose maximum reaches L are staged through LDS and their
//       passing elements become candidates (composite key, value descending
//       then index ascending), appended by wave-level stream compaction
//       (ballot + mbcnt) to a per-wave LDS region of 256 slots;
//     - if a region overflows (heavy ties), tie_select picks exactly k
//       candidates instead: the k-th key by bisection counting from
//       registers, then the first elements of that key in slot order.
//   Selection compacts the candidates, sorts 64- or 128-element runs with a
//   wave64 bitonic network and merges runs with bitonic merge-and-discard
//   (tx_wave_sort.h), giving the segment's sorted top-128.
//   Kernel B, seg_merge_kernel (only when nseg > 1, or over lists gathered
//   from vocabulary shards): one 4-wave workgroup per row loads every list at
//   once, merges them (merge-and-discard per wave, then a tree through LDS)
//   and writes (values, indices), the merged list, or runs the sampler tail.
//   The kernel boundary orders the workspace writes before the reads, so no
//   device-scope fence (an L2 write-back on gfx950) is ever issued.
#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "tallax_hip.h"
#include "tx_block_sort.h"
#include "tx_common.h"
#include "tx_host.h"
#include "tx_math.h"
#include "tx_sample.h"
#include "tx_scan.h"
#include "tx_wave_sort.h"

namespace tx {

constexpr int kNT = 256;                   // threads per segment workgroup: 4 wave64s
constexpr int kNTRow = 512;                // threads per whole-row workgroup: 8 wave64s, 2 per SIMD
constexpr int kMaxK = 128;                 // the reference's limit (top_k.py:438-439)
constexpr int kRun = 128;                  // list length handed between kernels
constexpr int kMaxSeg = 32;
constexpr int kTargetBlocks = 1024;        // ~4 workgroups per CU on 256 CUs
constexpr int kPartsMaxBlocks = 512;       // whole-row parts: two rounds of one workgroup per CU at most

struct SelArgs {
  const void* x;
  int64_t rows, cols;
  int k;
  int nseg;
  int64_t vps;  // 16-byte vectors per segment
  // top-k outputs
  void* out_vals;
  int32_t* out_idx;
  const int32_t* k_rows;  // optional: positions >= k_rows[row] get replace_in_dtype
  // segment lists: rows * nseg * kRun composites
  uint64_t* ws_lists;
  int lists_only;  // write the segment list even when a row is one segment
  int64_t col_offset;   // added to every column index of a written list (a vocabulary shard's first column)
  int64_t part_cols;    // whole-row kernel on row parts: row r of the [np rows, cols / np] view adds (r % np) * part_cols
  int nparts;
  int list_k;           // whole-row kernel: places of the row's (or part's) list that are read (64; 0: all 128)
  uint64_t* out_lists;  // merge kernel, lists_only: the merged list of each row, [rows][128]
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

// waves per workgroup and candidate slots per wave
template <int NT>
struct Geo {
  static constexpr int NW = NT / kWave;
  static constexpr int WCAP = 256;
};
constexpr int kStage = 6;                  // flagged 16-byte vectors staged per thread

// ---------------------------------------------------------------------------
// Per-dtype selection traits.
//
// Canonical keys order values the way select_key does (-0 == +0, NaN lowest).
// Raw keys, used only by the streaming filter, skip the canonicalisation:
// raw(x) = bits ^ (sign ? all-ones : sign-bit) is monotone in value except
// that -0 sits one below +0 and positive NaNs sit above +inf; raw_thr()
// turns a canonical threshold into a raw one that passes every element the
// canonical one does (positive NaNs become harmless extra candidates).
//
// bf16: canonical keys are 16 bits and a segment has < 65536 elements, so a
// candidate composite is one u32: key << 16 | (0xFFFF - segment-local index).
// f32: composite = canonical key << 32 | ~row index (u64).
// ---------------------------------------------------------------------------
template <int DT, bool WIDE>
struct Sel;

template <>
struct Sel<kBF16, false> {
  using Comp = uint32_t;
  static constexpr uint32_t kRawPosInf = 0xFF80u;
  __device__ static __forceinline__ uint32_t canon(uint32_t h) {  // h: bf16 bits
    const uint32_t a = h & 0x7FFFu;
    uint32_t k = (h & 0x8000u) ? (~h & 0xFFFFu) : (h | 0x8000u);
    k = a == 0u ? 0x8000u : k;
    k = a > 0x7F80u ? 0u : k;
    return k;
  }
  __device__ static __forceinline__ Comp comp(uint32_t h, uint32_t lidx) {
    return (canon(h) << 16) | (0xFFFFu - lidx);
  }
  __device__ static __forceinline__ uint32_t comp_key(Comp c) { return c >> 16; }
  // canonical key of a raw filter key (positive-NaN raw keys are handled by the caller)
  __device__ static __forceinline__ uint32_t raw_to_canon(uint32_t r) {
    return r == 0x7FFFu ? 0x8000u : (r < 0x007Fu ? 0u : r);
  }
  __device__ static __forceinline__ uint32_t raw_thr(uint32_t thr) {  // thr >= 1
    return thr == 0x8000u ? 0x7FFFu : thr;
  }
  __device__ static __forceinline__ uint64_t to_global(Comp c, int64_t seg_e0) {
    if (c == 0u) return 0ull;
    const uint32_t k16 = c >> 16;
    const uint32_t key = k16 == 0u ? 1u : (k16 >= 0x8000u ? (k16 << 16) : ((k16 << 16) | 0xFFFFu));
    return make_comp(key, (uint32_t)(seg_e0 + (int64_t)(0xFFFFu - (c & 0xFFFFu))));
  }
};

// bf16 in workgroups of more than 65535 elements: same canonical 16-bit keys,
// composite = key << 32 | ~row index (u64).
template <>
struct Sel<kBF16, true> {
  using Comp = uint64_t;
  static constexpr uint32_t kRawPosInf = 0xFF80u;
  __device__ static __forceinline__ uint32_t canon(uint32_t h) { return Sel<kBF16, false>::canon(h); }
  __device__ static __forceinline__ Comp comp(uint32_t h, uint32_t gidx) {
    return ((uint64_t)canon(h) << 32) | (uint64_t)(~gidx);
  }
  __device__ static __forceinline__ uint32_t comp_key(Comp c) { return (uint32_t)(c >> 32); }
  __device__ static __forceinline__ uint32_t raw_to_canon(uint32_t r) { return Sel<kBF16, false>::raw_to_canon(r); }
  __device__ static __forceinline__ uint32_t raw_thr(uint32_t thr) { return Sel<kBF16, false>::raw_thr(thr); }
  __device__ static __forceinline__ uint64_t to_global(Comp c, int64_t) {
    if (c == 0ull) return 0ull;
    const uint32_t k16 = (uint32_t)(c >> 32);
    const uint32_t key = k16 == 0u ? 1u : (k16 >= 0x8000u ? (k16 << 16) : ((k16 << 16) | 0xFFFFu));
    return make_comp(key, ~(uint32_t)c);
  }
};

template <bool WIDE>
struct Sel<kF32, WIDE> {
  using Comp = uint64_t;
  static constexpr uint32_t kRawPosInf = 0xFF800000u;
  __device__ static __forceinline__ uint32_t canon(uint32_t b) { return select_key(b); }
  __device__ static __forceinline__ Comp comp(uint32_t b, uint32_t gidx) { return make_comp(select_key(b), gidx); }
  __device__ static __forceinline__ uint32_t comp_key(Comp c) { return (uint32_t)(c >> 32); }
  __device__ static __forceinline__ uint32_t raw_to_canon(uint32_t r) {
    return r == 0x7FFFFFFFu ? 0x80000000u : (r < 0x007FFFFFu ? 1u : r);
  }
  __device__ static __forceinline__ uint32_t raw_thr(uint32_t thr) {
    return thr <= 1u ? 0u : (thr == 0x80000000u ? 0x7FFFFFFFu : thr);
  }
  __device__ static __forceinline__ uint64_t to_global(Comp c, int64_t) { return c; }
};

template <typename C, int NT>
struct SegShared {
  static constexpr int NW = Geo<NT>::NW, WCAP = Geo<NT>::WCAP;
  C cand[NW * WCAP];  // wave w owns cand[w * WCAP, (w + 1) * WCAP)
  C scratch[NW * kRun];
  C list[kRun];
  uint64_t list64[kRun];
  float samp_g[kRun];  // sampler: Gumbel noise of the top-128
  uint32_t wl[NW];
  int red[NW];
  int wc[NW];  // per-wave candidate counts
};

// sh.list <- the 128 largest candidates of all wave regions (counts cnt[w] in LDS),
// descending, zero padded.  Sets of at most 64 per wave use chunk_select;
// larger ones are sorted per wave region in runs of 128 and the per-wave
// lists merged as a binary tree (log2(waves) levels).
// Chunked selection for candidate sets of at most 64 per wave: the
// candidates are compacted into sh.scratch, wave w sorts chunk w (64, one per
// lane), and the sorted chunks are merged pairwise: 64 + 64 -> 128 by a
// bitonic merge, then 128-runs by merge-and-discard, until one run is left.
template <typename C, int NT>
__device__ __forceinline__ void chunk_select(SegShared<C, NT>& sh, const int* cnt, int total) {
  constexpr int NW = Geo<NT>::NW, WCAP = Geo<NT>::WCAP;
  const int tid = threadIdx.x, w = tid / kWave, l = lane_id();
  int off = 0;
#pragma unroll
  for (int q = 0; q < NW; ++q) off += q < w ? (cnt[q] < WCAP ? cnt[q] : WCAP) : 0;
  const int cw = cnt[w] < WCAP ? cnt[w] : WCAP;
  for (int i = l; i < cw; i += kWave) sh.scratch[off + i] = sh.cand[w * WCAP + i];
  __syncthreads();
  const int nch = (total + kWave - 1) / kWave;  // 64-chunks, <= NW
  if (w < nch) {
    const int i = w * kWave + l;
    const C v = wave_sort64_desc<C>(i < total ? sh.scratch[i] : (C)0);
    sh.scratch[i] = v;
  }
  __syncthreads();
  // level 0: chunks 2r, 2r+1 -> 128-run r (stored in place at scratch + 128 r)
  const int nrun = (nch + 1) / 2;
  if (w < nrun) {
    C c[2];
    c[0] = sh.scratch[2 * w * kWave + l];
    c[1] = 2 * w + 1 < nch ? sh.scratch[(2 * w + 1) * kWave + (kWave - 1 - l)] : (C)0;  // reversed: bitonic
    wave_bitonic_merge128_desc(c);
    sh.scratch[w * kRun + l] = c[0];
    sh.scratch[w * kRun + kWave + l] = c[1];
  }
  __syncthreads();
  for (int st = 1; st < nrun; st <<= 1) {
    if ((w & (2 * st - 1)) == 0 && w + st < nrun) {
      C acc[2] = {sh.scratch[w * kRun + l], sh.scratch[w * kRun + kWave + l]};
      const C b[2] = {sh.scratch[(w + st) * kRun + l], sh.scratch[(w + st) * kRun + kWave + l]};
      wave_merge128_desc(acc, b);
      sh.scratch[w * kRun + l] = acc[0];
      sh.scratch[w * kRun + kWave + l] = acc[1];
    }
    __syncthreads();
  }
  for (int i = tid; i < kRun; i += NT) sh.list[i] = nrun > 0 ? sh.scratch[i] : (C)0;
  __syncthreads();
}

template <typename C, int NT>
__device__ __forceinline__ void block_select(SegShared<C, NT>& sh, const int* cnt) {
  constexpr int NW = Geo<NT>::NW, WCAP = Geo<NT>::WCAP;
  int total = 0;
#pragma unroll
  for (int q = 0; q < NW; ++q) total += cnt[q] < WCAP ? cnt[q] : WCAP;
  if (total <= NW * kWave) {
    chunk_select(sh, cnt, total);
    return;
  }
  const int w = threadIdx.x / kWave, l = lane_id();
  const int cw = cnt[w] < WCAP ? cnt[w] : WCAP;
  const C* reg = sh.cand + w * WCAP;
  C acc[2] = {0, 0};
  for (int r = 0; r * kRun < cw; ++r) {
    C c[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = r * kRun + h * kWave + l;
      c[h] = i < cw ? reg[i] : (C)0;
    }
    wave_sort128_desc(c);
    if (r == 0) {
      acc[0] = c[0];
      acc[1] = c[1];
    } else {
      wave_merge128_desc(acc, c);
    }
  }
#pragma unroll
  for (int st = 1; st < NW; st <<= 1) {
    if ((w & (2 * st - 1)) == st) {
      sh.scratch[w * kRun + l] = acc[0];
      sh.scratch[w * kRun + kWave + l] = acc[1];
    }
    __syncthreads();
    if ((w & (2 * st - 1)) == 0) {
      const C b[2] = {sh.scratch[(w + st) * kRun + l], sh.scratch[(w + st) * kRun + kWave + l]};
      wave_merge128_desc(acc, b);
    }
  }
  if (w == 0) {
    sh.list[l] = acc[0];
    sh.list[kWave + l] = acc[1];
  }
  __syncthreads();
}

// Wave-level stream compaction: lanes with `pred` append `comp` to their
// wave's region at wcnt + (rank among active lanes).  `wcnt` is wave-uniform;
// entries beyond the region are counted but not stored.
template <int WCAP, typename C>
__device__ __forceinline__ void wave_append(bool pred, C comp, C* reg, int& wcnt) {
  const uint64_t m = __ballot(pred);
  if (m) {
    if (pred) {
      const int off = wcnt + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                            __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
      if (off < WCAP) reg[off] = comp;
    }
    wcnt += (int)__popcll(m);
  }
}

typedef short short2_t __attribute__((ext_vector_type(2)));
typedef unsigned short ushort2_t __attribute__((ext_vector_type(2)));

// Raw keys of the two bf16 values of a dword, packed (v_pk_ashrrev_i16 + xor/or).
__device__ __forceinline__ uint32_t raw_key2_bf16(uint32_t w) {
  const short2_t m = __builtin_bit_cast(short2_t, w) >> (short2_t){15, 15};
  return w ^ (__builtin_bit_cast(uint32_t, m) | 0x80008000u);
}
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(ushort2_t, a),
                                                                __builtin_bit_cast(ushort2_t, b)));
}
__device__ __forceinline__ uint32_t pk_sub_sat_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat(__builtin_bit_cast(ushort2_t, a),
                                                                    __builtin_bit_cast(ushort2_t, b)));
}
__device__ __forceinline__ uint32_t raw_key_f32(uint32_t b) {
  return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}
__device__ __forceinline__ uint32_t dword_of(const uint4 v, int d) {
  const uint32_t lo = (d & 1) ? v.y : v.x;
  const uint32_t hi = (d & 1) ? v.w : v.z;
  return (d & 2) ? hi : lo;
}
// Element q of a 16-byte vector as the value the select keys expect
// (bf16: its 16 bits, f32: its 32 bits); q may be a run-time value.
template <int DT>
__device__ __forceinline__ uint32_t elem_bits(const uint4 v, int q) {
  if (DT == kBF16) {
    const uint32_t w = dword_of(v, q >> 1);
    return (q & 1) ? (w >> 16) : (w & 0xFFFFu);
  }
  return dword_of(v, q);
}

// A row's sampler parameters, loaded when the kernel starts so that their
// memory latency is not paid in the tail.
struct RowParams {
  int kr;           // top_k[row]
  float top_p;
  float temp;
  uint32_t k0, k1;  // threefry key
  uint32_t row_ctr;  // row + dim0_offset
  uint32_t vocab;
  float replace_in_dtype, replace_f32;
};
template <bool SAMPLE>
__device__ __forceinline__ RowParams load_row_params(const SelArgs& a, int64_t row) {
  RowParams rp = {0, 0.0f, 0.0f, 0u, 0u, 0u, 0u, 0.0f, 0.0f};
  if (SAMPLE) {
    rp.kr = a.top_k[row];
    rp.top_p = a.top_p[row];
    rp.temp = a.temperature[row];
    rp.k0 = a.rng_key[0];
    rp.k1 = a.rng_key[1];
    rp.row_ctr = (uint32_t)(row + a.dim0_offset);
    rp.vocab = (uint32_t)a.cols;
    rp.replace_in_dtype = a.replace_in_dtype;
    rp.replace_f32 = a.replace_f32;
  }
  return rp;
}

// Outputs of one row from its sorted top-128 list (in LDS).  Called by every
// thread of the workgroup; sg is a 128-float LDS buffer (sampler only).
template <int DT, bool SAMPLE>
__device__ void finalize_row(const SelArgs& a, int64_t row, const uint64_t* list, float* sg, const RowParams& rp) {
  using T = ElemT<DT>;
  const uint32_t inel = ineligible_key_max(DT);
  if (!SAMPLE) {
    const char* rowp = (const char*)a.x + (size_t)(row * a.cols) * T::ES;
    for (int i = threadIdx.x; i < a.k; i += blockDim.x) {
      const uint64_t c = list[i];
      const uint32_t kk = comp_key(c);
      const int32_t idx = comp_idx(c);
      // the key fixes the value except the sign of a zero: only zeros are reloaded
      uint32_t b = kk > inel ? (kk == 0x80000000u ? T::load_bits(rowp, idx) : key_to_bits(kk)) : T::kMinBits;
      if (a.k_rows && i >= a.k_rows[row]) b = __float_as_uint(a.replace_in_dtype);
      T::store(a.out_vals, row * a.k + i, b);
      a.out_idx[row * a.k + i] = idx;
    }
    return;
  }
  // value at position p of the top-128, positions >= top_k[row] replaced
  const int kr = rp.kr;
  auto value_at = [&](int p) -> float {
    const uint32_t kk = comp_key(list[p]);
    const float val = __uint_as_float(kk > inel ? key_to_bits(kk) : T::kMinBits);
    return p < kr ? val : rp.replace_in_dtype;
  };
  const uint32_t row_ctr = rp.row_ctr;
  const uint32_t k0 = rp.k0, k1 = rp.k1;
  const int tid = threadIdx.x, l = lane_id();
  // Waves 1-2 compute the Gumbel noise of the 128 candidates while wave 0
  // finds the top-p threshold (a 64-thread block does both in wave 0).
  const bool split = blockDim.x >= 3 * kWave;
  if (split && tid >= kWave && tid < kWave + kMaxK) {
    const int p = tid - kWave;
    sg[p] = candidate_noise(k0, k1, row_ctr, rp.vocab, comp_idx(list[p]));
  }
  float v[2], e[2], g[2];
  int32_t id[2];
  float thr = 0.0f;
  if (tid < kWave) {
    const float v0 = value_at(0);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int p = h * kWave + l;
      v[h] = value_at(p);
      id[h] = comp_idx(list[p]);
      e[h] = candidate_exp(v[h], v0);
      if (!split) g[h] = candidate_noise(k0, k1, row_ctr, rp.vocab, id[h]);
    }
    thr = top_p_threshold(v, e, kMaxK, rp.top_p);
  }
  if (split) __syncthreads();
  if (tid < kWave) {
    if (split) {
      g[0] = sg[l];
      g[1] = sg[kWave + l];
    }
    const int32_t tok = gumbel_argmax(v, id, g, kMaxK, thr, rp.temp, rp.replace_f32);
    if (l == 0) a.out_tokens[row] = tok;
  }
}

// ---------------------------------------------------------------------------
// Views of the raw bits used to bound vector maxima cheaply:
//   signed view   f32 bits as int32, bf16 halves as int16: monotone over
//                 non-negative values (positive NaNs sit above +inf), every
//                 negative value is below +0.  One integer max per element
//                 pair, so it serves rows whose threshold is positive.
//   ordered view  bits ^ (sign ? 0x7F..F : 0): monotone over all values
//                 (-0 one below +0, positive NaNs above +inf, negative NaNs
//                 below -inf); canonical key = ordered + 2^(bits-1), except
//                 -0 (ordered -1) whose key is that of +0.
// Slots outside the row or the segment hold all-ones (a negative NaN): -1 in
// the signed view and the minimum of the ordered view.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pk_max_i16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(short2_t, a),
                                                                __builtin_bit_cast(short2_t, b)));
}
__device__ __forceinline__ int32_t imax32(int32_t a, int32_t b) { return a > b ? a : b; }
// larger of the two signed halves, sign-extended
__device__ __forceinline__ int32_t hmax_i16(uint32_t m) {
  return imax32((int32_t)(int16_t)(m & 0xFFFFu), (int32_t)(int16_t)(m >> 16));
}
__device__ __forceinline__ uint32_t ord2_bf16(uint32_t w) {
  const short2_t m = __builtin_bit_cast(short2_t, w) >> (short2_t){15, 15};
  return w ^ (__builtin_bit_cast(uint32_t, m) & 0x7FFF7FFFu);
}
__device__ __forceinline__ uint32_t ord_f32(uint32_t b) {
  return b ^ ((uint32_t)((int32_t)b >> 31) & 0x7FFFFFFFu);
}
// signed-view maximum of a 16-byte vector (sign-extended)
template <int DT>
__device__ __forceinline__ int32_t vec_smax(const uint4 v) {
  if (DT == kBF16) return hmax_i16(pk_max_i16(pk_max_i16(v.x, v.y), pk_max_i16(v.z, v.w)));
  return imax32(imax32((int32_t)v.x, (int32_t)v.y), imax32((int32_t)v.z, (int32_t)v.w));
}
// ordered-view maximum of a 16-byte vector
template <int DT>
__device__ __forceinline__ int32_t vec_omax(const uint4 v) {
  if (DT == kBF16)
    return hmax_i16(pk_max_i16(pk_max_i16(ord2_bf16(v.x), ord2_bf16(v.y)),
                               pk_max_i16(ord2_bf16(v.z), ord2_bf16(v.w))));
  return imax32(imax32((int32_t)ord_f32(v.x), (int32_t)ord_f32(v.y)),
                imax32((int32_t)ord_f32(v.z), (int32_t)ord_f32(v.w)));
}

// ---------------------------------------------------------------------------
// Heavy ties (a candidate region overflowed, e.g. constant rows or rows of
// -inf but a few): the k candidates are chosen exactly.  The k-th largest
// canonical key K comes from a bisection over the key bits, counting
// straight from registers (one pass over the thread's elements and one
// block sum per bit); the elements above K are appended, then the first
// k - #above of key K in slot order: vector j of every thread (threads in
// order) precedes vector j + 1, so one block scan per vector index until
// enough are taken (usually at j = 0).  The append passes take the vectors
// through the thread's own stage slots, kStage at a time, with one loop body
// per vector.
//   It is a separate, non-inlined function that loads the segment again, so
// that its register needs do not weigh on the selection kernel's common path.
//   The counts use the raw-key order, which equals the canonical order but
// for -0 (one below +0), positive NaNs (above +inf) and negative NaNs and
// dead slots (below -inf): per-thread counts of the first two correct the
// sums, and probes below the key of -inf count every live element, since no
// canonical key lies between a NaN's and -inf's.
// Returns this wave's number of appended candidates.  Every thread calls it.
// ---------------------------------------------------------------------------
template <int DT, int MAXV, int NT, int SG = kStage>
__device__ __attribute__((noinline)) int tie_select(const uint4* base, int64_t s0, int64_t s1, int lbase,
                                                    int live_lo, int live_hi, uint32_t gbase, int k,
                                                    typename Sel<DT, (NT * MAXV * ElemT<DT>::VEC > 65535)>::Comp* reg,
                                                    int* red, uint4* stage) {
  using T = ElemT<DT>;
  constexpr bool kWide = NT * MAXV * T::VEC > 65535;
  using S = Sel<DT, kWide>;
  using C = typename S::Comp;
  constexpr bool kBF = DT == kBF16;
  constexpr int VEC = T::VEC, NW = Geo<NT>::NW, WCAP = Geo<NT>::WCAP;
  constexpr uint32_t kZeroKey = kBF ? 0x8000u : 0x80000000u;     // canonical key of +-0
  constexpr uint32_t kNaNKey = kBF ? 0u : 1u;                     // canonical key of every NaN
  constexpr uint32_t kNegInfKey = kBF ? 0x007Fu : 0x007FFFFFu;    // canonical key of -inf
  constexpr int kKeyBits = kBF ? 16 : 32;
  const int tid = threadIdx.x;
  auto elem_id = [&](int lidx) -> uint32_t { return (kBF && !kWide) ? (uint32_t)lidx : gbase + (uint32_t)lidx; };
  auto live_bits = [&](int li0) -> uint32_t {
    uint32_t m = 0;
#pragma unroll
    for (int q = 0; q < VEC; ++q) m |= (li0 + q >= live_lo && li0 + q < live_hi ? 1u : 0u) << q;
    return m;
  };
  // the segment again, slots outside the row as all-ones
  uint4 raw[MAXV];
#pragma unroll
  for (int j = 0; j < MAXV; ++j) {
    const int64_t v = s0 + (int64_t)j * NT + tid;
    raw[j] = v < s1 ? base[v] : make_uint4(~0u, ~0u, ~0u, ~0u);
  }
  int nlive = 0, nposnan = 0, nnegzero = 0;
#pragma unroll
  for (int j = 0; j < MAXV; ++j) {
    const uint32_t lm = live_bits(lbase + j * NT * VEC);
    uint32_t d[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // dead slots become all-ones
      if (kBF) {
        d[i] |= ((lm >> (2 * i)) & 1u) ? 0u : 0x0000FFFFu;
        d[i] |= ((lm >> (2 * i + 1)) & 1u) ? 0u : 0xFFFF0000u;
      } else {
        d[i] |= ((lm >> i) & 1u) ? 0u : ~0u;
      }
    }
    const uint4 v = make_uint4(d[0], d[1], d[2], d[3]);
#pragma unroll
    for (int q = 0; q < VEC; ++q) {
      const uint32_t bq = elem_bits<DT>(v, q);
      const bool live = (lm >> q) & 1u;
      nlive += live ? 1 : 0;
      nposnan += live && bq > (kBF ? 0x7F80u : 0x7F800000u) && bq < kZeroKey ? 1 : 0;
      nnegzero += live && bq == kZeroKey ? 1 : 0;
    }
    // from here on the raw keys (dead slots: 0)
#pragma unroll
    for (int i = 0; i < 4; ++i) d[i] = kBF ? raw_key2_bf16(d[i]) : raw_key_f32(d[i]);
    raw[j] = make_uint4(d[0], d[1], d[2], d[3]);
  }
  // canonical key from a raw key: NaNs (above +inf or below -inf) and -0 differ
  auto canon_of = [&](uint32_t rk) -> uint32_t {
    const uint32_t kc = rk == kZeroKey - 1u ? kZeroKey : rk;
    return rk > (kBF ? 0xFF80u : 0xFF800000u) || rk < kNegInfKey ? kNaNKey : kc;
  };
  // composite of an element from its canonical key and slot, as S::comp builds it
  auto comp_of = [&](uint32_t kc, int lidx) -> C {
    if constexpr (sizeof(C) == 4) return (C)((kc << 16) | (0xFFFFu - (uint32_t)lidx));
    else return (C)(((uint64_t)kc << 32) | (uint64_t)(~elem_id(lidx)));
  };
  // live elements whose canonical key is >= P
  auto count_ge = [&](uint32_t P) -> int {
    if (P <= kNaNKey) return nlive;
    const uint32_t pr = P < kNegInfKey ? kNegInfKey : P;
    int c = 0;
    if constexpr (kBF) {
      // both halves at once: sat(rk - (pr - 1)) is 0 exactly when rk < pr; min(., 1) counts
      const ushort2_t pm1 = __builtin_bit_cast(ushort2_t, (pr - 1u) * 0x10001u);
      const ushort2_t one = __builtin_bit_cast(ushort2_t, 0x00010001u);
      ushort2_t acc = __builtin_bit_cast(ushort2_t, 0u);
#pragma unroll
      for (int j = 0; j < MAXV; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const ushort2_t rk = __builtin_bit_cast(ushort2_t, dword_of(raw[j], i));
          acc += __builtin_elementwise_min(__builtin_elementwise_sub_sat(rk, pm1), one);
        }
      }
      const uint32_t a2 = __builtin_bit_cast(uint32_t, acc);
      c = (int)((a2 & 0xFFFFu) + (a2 >> 16));
    } else {
#pragma unroll
      for (int j = 0; j < MAXV; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) c += dword_of(raw[j], i) >= pr ? 1 : 0;
      }
    }
    return c - nposnan + (P == kZeroKey ? nnegzero : 0);
  };
  uint32_t K = 0;
#pragma unroll 1
  for (int b = kKeyBits - 1; b >= 0; --b) {
    const uint32_t probe = K | (1u << b);
    if (block_sum<NW>(count_ge(probe), red) >= k) K = probe;
  }
  const int above = block_sum<NW>(count_ge(K + 1u), red);  // K < the largest key: no wrap
  int rest = k - above;                                    // >= 1 elements of key K
  int wcnt = 0;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
    for (int c = 0; c < (MAXV + SG - 1) / SG; ++c) {
      if (pass == 1 && rest <= 0) break;
#pragma unroll
      for (int u = 0; u < SG; ++u)
        if (c * SG + u < MAXV) stage[u * NT + tid] = raw[c * SG + u];
#pragma unroll 1
      for (int u = 0; u < SG && c * SG + u < MAXV; ++u) {
        if (pass == 1 && rest <= 0) break;
        const int li0 = lbase + (c * SG + u) * NT * VEC;
        const uint4 vv = stage[u * NT + tid];
        const uint32_t lm = live_bits(li0);
        uint32_t mask = 0;
        if (pass == 0) {  // above K
#pragma unroll
          for (int q = 0; q < VEC; ++q)
            mask |= (((lm >> q) & 1u) && canon_of(elem_bits<DT>(vv, q)) > K ? 1u : 0u) << q;
        } else {  // key K, the first `rest` in slot order
          uint32_t eq = 0;
#pragma unroll
          for (int q = 0; q < VEC; ++q)
            eq |= (((lm >> q) & 1u) && canon_of(elem_bits<DT>(vv, q)) == K ? 1u : 0u) << q;
          int total = 0;
          const int before = block_exscan<NW>(__popc(eq), red, total);
#pragma unroll
          for (int q = 0; q < VEC; ++q)
            mask |= (((eq >> q) & 1u) && before + __popc(eq & ((1u << q) - 1u)) < rest ? 1u : 0u) << q;
          rest -= total;
        }
        for (;;) {
          const bool hc = mask != 0u;
          if (!__ballot(hc)) break;
          C cm = 0;
          if (hc) {
            const int e = __builtin_ctz(mask);
            mask &= mask - 1u;
            cm = comp_of(canon_of(elem_bits<DT>(vv, e)), li0 + e);
          }
          wave_append<WCAP>(hc, cm, reg, wcnt);
        }
      }
    }
  }
  return wcnt;
}

// ---------------------------------------------------------------------------
// Kernel A: one workgroup per (segment, row).  The segment (MAXV 16-byte
// vectors per thread) is loaded into registers with every load issued up
// front; a per-thread maximum bounds the k-th key from below (L); vectors
// that may hold an element >= L are staged in LDS and their passing elements
// appended to per-wave candidate regions; one block selection gives the
// sorted top-128.  Candidate regions that overflow (heavy ties) switch to an
// exact bisection on the composite key over the same staged rounds.
// ---------------------------------------------------------------------------
template <int DT, int MAXV, int NT, bool SAMPLE>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(NT == kNTRow ? 2 : 4, 8)))
void seg_select_kernel(SelArgs a) {
  using T = ElemT<DT>;
  constexpr bool kWide = NT * MAXV * T::VEC > 65535;  // block-local bf16 indices need > 16 bits
  using S = Sel<DT, kWide>;
  using C = typename S::Comp;
  constexpr bool kBF = DT == kBF16;
  constexpr int VEC = T::VEC, ES = T::ES;
  constexpr int NW = Geo<NT>::NW, WCAP = Geo<NT>::WCAP;
  constexpr uint32_t kZeroKey = kBF ? 0x8000u : 0x80000000u;  // canonical key of +-0
  constexpr int32_t kPosInf = kBF ? 0x7F80 : 0x7F800000;      // +inf bits (signed / ordered view)
  constexpr int32_t kOrdNegInf = kBF ? -32641 : (int32_t)0x807FFFFFu;  // ordered view of -inf
  __shared__ SegShared<C, NT> sh;
  __shared__ uint4 stage[kStage * NT];  // staged vectors, slot-major
  const int tid = threadIdx.x;
  const int w = tid / kWave, l = lane_id();
  const int64_t row = blockIdx.x / (unsigned)a.nseg;  // one-dimensional grid: rows beyond 65535
  const int seg = (int)(blockIdx.x - row * a.nseg);
  const int k = a.k;
  const RowParams rp = load_row_params<SAMPLE>(a, row);

  const char* rowp = (const char*)a.x + (size_t)(row * a.cols) * ES;
  const RowVec<ES> rv(rowp);
  const int64_t nv = (a.cols + rv.mis + VEC - 1) / VEC;
  const int64_t s0 = (int64_t)seg * a.vps;
  const int64_t s1 = s0 + a.vps < nv ? s0 + a.vps : nv;
  const int64_t seg_e0 = s0 * VEC - rv.mis;  // element index of the segment's first slot
  C* reg = sh.cand + w * WCAP;

  uint4 raw[MAXV];
#pragma unroll
  for (int j = 0; j < MAXV; ++j) {
    const int64_t v = s0 + (int64_t)j * NT + tid;
    raw[j] = v < s1 ? load_once(rv.base + v) : make_uint4(~0u, ~0u, ~0u, ~0u);
  }
  // Segment-local slot index of (j, q): lbase + j * NT * VEC + q.  Live slots
  // (inside the row and the segment) are those in [live_lo, live_hi).
  const int lbase = tid * VEC;
  const int64_t seg_elems = (s1 - s0) * VEC;
  const int live_lo = seg_e0 < 0 ? (int)(-seg_e0) : 0;
  const int live_hi = (int)(a.cols - seg_e0 < seg_elems ? a.cols - seg_e0 : seg_elems);
  const uint32_t gbase = (uint32_t)seg_e0;  // row index = gbase + local index (mod 2^32)
  auto elem_id = [&](int lidx) -> uint32_t { return (kBF && !kWide) ? (uint32_t)lidx : gbase + (uint32_t)lidx; };
  auto vec_full = [&](int j) -> bool {
    const int li0 = lbase + j * NT * VEC;
    return li0 >= live_lo && li0 + VEC <= live_hi;
  };
  auto vec_dead = [&](int j) -> bool {
    const int li0 = lbase + j * NT * VEC;
    return li0 >= live_hi || li0 + VEC <= live_lo;
  };
  // live-slot mask of the vector at local slot li0 (bit q: slot li0 + q is live)
  auto live_mask = [&](int li0) -> uint32_t {
    uint32_t m = 0;
#pragma unroll
    for (int q = 0; q < VEC; ++q) m |= (li0 + q >= live_lo && li0 + q < live_hi ? 1u : 0u) << q;
    return m;
  };
  // dead slots of partial vectors (first / last of a row) become all-ones
#pragma unroll
  for (int j = 0; j < MAXV; ++j) {
    if (!vec_full(j) && !vec_dead(j)) {
      const uint32_t lm = live_mask(lbase + j * NT * VEC);
      uint32_t d[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (kBF) {
          d[i] |= ((lm >> (2 * i)) & 1u) ? 0u : 0x0000FFFFu;
          d[i] |= ((lm >> (2 * i + 1)) & 1u) ? 0u : 0xFFFF0000u;
        } else {
          d[i] |= ((lm >> i) & 1u) ? 0u : ~0u;
        }
      }
      raw[j] = make_uint4(d[0], d[1], d[2], d[3]);
    }
  }

  // ---- thread maximum as a canonical key ---------------------------------------
  int32_t smax = kBF ? -32768 : (int32_t)0x80000000u;
#pragma unroll
  for (int j = 0; j < MAXV; ++j) smax = imax32(smax, vec_smax<DT>(raw[j]));
  uint32_t tmax;
  if (smax >= 0 && smax <= kPosInf) {
    tmax = (uint32_t)smax | kZeroKey;
  } else {  // no non-negative element, or a positive NaN: use the ordered view
    int32_t omax = kBF ? -32768 : (int32_t)0x80000000u;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) omax = imax32(omax, vec_omax<DT>(raw[j]));
    if (omax < kOrdNegInf) {
      tmax = 0;  // only NaNs / dead slots: 0 is a valid (low) bound
    } else if (omax <= kPosInf) {
      tmax = omax == -1 ? kZeroKey : (uint32_t)omax + kZeroKey;
    } else {  // positive NaN: canonical maximum slot by slot
      tmax = 0;
#pragma unroll
      for (int j = 0; j < MAXV; ++j) {
        const int li0 = lbase + j * NT * VEC;
#pragma unroll 1
        for (int q = 0; q < VEC; ++q) {
          const uint32_t kk = S::canon(elem_bits<DT>(raw[j], q));
          tmax = (li0 + q >= live_lo && li0 + q < live_hi && kk > tmax) ? kk : tmax;
        }
      }
    }
  }

  // ---- lower bound L: at least k live elements are >= L --------------------
  const uint32_t srt = wave_sort64_u32_desc(tmax);
  const uint32_t wl = readlane_u32(srt, (k + NW - 1) / NW - 1);  // this wave's quota of maxima
  if (l == 0) sh.wl[w] = wl;
  __syncthreads();
  uint32_t L = sh.wl[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) L = sh.wl[i] < L ? sh.wl[i] : L;
  const uint32_t thr = kBF ? L : (L > 1u ? L : 1u);  // candidates: live elements with canonical key >= thr

  // ---- flags: vectors whose maximum may reach thr ------------------------------
  const bool nan_level = kBF ? thr == 0u : thr <= 1u;  // thr admits NaNs: every live vector
  const bool pos_thr = !nan_level && thr > kZeroKey;   // positive threshold: signed view
  const int32_t st = (int32_t)(thr - kZeroKey);        // its bits, when positive
  uint32_t fl = 0;
  if (pos_thr) {
#pragma unroll
    for (int j = 0; j < MAXV; ++j) fl |= (vec_smax<DT>(raw[j]) >= st ? 1u : 0u) << j;
  } else {
    const int32_t ot = nan_level ? (int32_t)0x80000000u : (thr == kZeroKey ? -1 : (int32_t)(thr - kZeroKey));
#pragma unroll
    for (int j = 0; j < MAXV; ++j) fl |= (!vec_dead(j) && vec_omax<DT>(raw[j]) >= ot ? 1u : 0u) << j;
  }
  const int nfl = __popc(fl);

  // ---- candidates -----------------------------------------------------------------
  // Flagged vectors are staged in LDS kStage at a time ("rounds"); each staged
  // element passes if it is live, its canonical key is >= thr and, with a
  // probe, its composite is >= probe.  Passing elements are appended to the
  // wave's region, or only counted (count_only).
  auto pass_mask = [&](const uint4 vv, int li0) -> uint32_t {
    uint32_t m = 0;
    if (pos_thr) {
      // positive threshold: st <= bits <= +inf in the signed view (NaNs excluded);
      // dead slots (all-ones, -1) fail
      const uint32_t span = (uint32_t)(kPosInf - st);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t x = dword_of(vv, d);
        if (kBF) {
          m |= ((uint32_t)((int32_t)(int16_t)(x & 0xFFFFu) - st) <= span ? 1u : 0u) << (2 * d);
          m |= ((uint32_t)(((int32_t)x >> 16) - st) <= span ? 1u : 0u) << (2 * d + 1);
        } else {
          m |= ((uint32_t)((int32_t)x - st) <= span ? 1u : 0u) << d;
        }
      }
      return m;
    }
#pragma unroll
    for (int q = 0; q < VEC; ++q) m |= (S::canon(elem_bits<DT>(vv, q)) >= thr ? 1u : 0u) << q;
    if (li0 < live_lo || li0 + VEC > live_hi) m &= live_mask(li0);
    return m;
  };
  auto rounds = [&](int& wcnt) {
#pragma unroll 1
    for (int first = 0;; first += kStage) {
      uint32_t slots = 0;
      int o = 0;
#pragma unroll
      for (int j = 0; j < MAXV; ++j) {
        if ((fl >> j) & 1u) {
          const int sl = o - first;
          if (sl >= 0 && sl < kStage) {
            stage[sl * NT + tid] = raw[j];
            slots |= (uint32_t)j << (5 * sl);
          }
          ++o;
        }
      }
      const int nst = nfl - first;
#pragma unroll 1
      for (int i = 0; i < kStage; ++i) {
        const bool have = i < nst;
        // a full region means the tie selection takes over: stop appending
        if (!__ballot(have) || wcnt > WCAP) break;
        uint32_t mask = 0;
        uint4 vv = make_uint4(0u, 0u, 0u, 0u);
        int li0 = 0;
        if (have) {
          vv = stage[i * NT + tid];
          li0 = lbase + (int)((slots >> (5 * i)) & 31u) * NT * VEC;
          mask = pass_mask(vv, li0);
        }
        for (;;) {
          const bool hc = mask != 0u;
          if (!__ballot(hc)) break;
          C cm = 0;
          if (hc) {
            const int e = __builtin_ctz(mask);
            mask &= mask - 1u;
            // the element, read back from its staged copy
            const uint32_t bits = kBF ? (uint32_t)((const uint16_t*)&stage[i * NT + tid])[e]
                                      : ((const uint32_t*)&stage[i * NT + tid])[e];
            cm = S::comp(bits, elem_id(li0 + e));
          }
          wave_append<WCAP>(hc, cm, reg, wcnt);
        }
      }
      if (!__ballot(nfl > first + kStage) || wcnt > WCAP) break;
    }
  };

  // Filter pass; exact tie selection when a region overflows.  Control flow
  // is block-uniform.
  {
    int wcnt = 0;
    rounds(wcnt);
    if (l == 0) sh.wc[w] = wcnt;
    __syncthreads();
    bool overflow = false;
#pragma unroll
    for (int q = 0; q < NW; ++q) overflow |= sh.wc[q] > WCAP;
    if (overflow) {
      // its block sums order the reads of sh.wc above before the write below
      wcnt = tie_select<DT, MAXV, NT>(rv.base, s0, s1, lbase, live_lo, live_hi, gbase, k, reg, sh.red, stage);
      if (l == 0) sh.wc[w] = wcnt;
      __syncthreads();
    }
  }

  block_select(sh, (const int*)sh.wc);
  for (int i = tid; i < kRun; i += NT) sh.list64[i] = S::to_global(sh.list[i], seg_e0);
  __syncthreads();
  if (a.nseg == 1 && !a.lists_only) {
    finalize_row<DT, SAMPLE>(a, row, sh.list64, sh.samp_g, rp);
  } else {
    uint64_t* dst = a.ws_lists + ((size_t)row * a.nseg + seg) * kRun;
    // ~(idx + off) = ~idx - off without a borrow into the key (idx + off < 2^31); empty slots stay 0
    for (int i = tid; i < kRun; i += NT) dst[i] = sh.list64[i] ? sh.list64[i] - (uint64_t)a.col_offset : 0ull;
  }
}

// ---------------------------------------------------------------------------
// Kernel B: one workgroup of kMergeNT threads per row merges the segment
// lists and finishes the row.  Wave w loads lists w, w + NW, ... all at once
// (they were written by other CUs, so every load is a full memory latency),
// folds them with merge-and-discard, and the per-wave lists are merged as a
// binary tree through LDS.
// ---------------------------------------------------------------------------
constexpr int kMergeNT = 256;
template <int DT, bool SAMPLE>
__global__ __launch_bounds__(kMergeNT) void seg_merge_kernel(SelArgs a) {
  constexpr int NW = kMergeNT / kWave;
  constexpr int PER = kMaxSeg / NW;  // lists per wave, at most
  __shared__ uint64_t tree[NW][kRun];
  __shared__ float sg[kRun];
  const int64_t row = blockIdx.x;
  const int w = threadIdx.x / kWave, l = lane_id();
  const uint64_t* src = a.ws_lists + (size_t)row * a.nseg * kRun;
  const RowParams rp = load_row_params<SAMPLE>(a, row);
  uint64_t b[PER][2];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int sgi = w + i * NW;
    b[i][0] = sgi < a.nseg ? src[sgi * kRun + l] : 0ull;
    b[i][1] = sgi < a.nseg ? src[sgi * kRun + kWave + l] : 0ull;
  }
  uint64_t acc[2] = {b[0][0], b[0][1]};
#pragma unroll
  for (int i = 1; i < PER; ++i) {
    if (w + i * NW < a.nseg) wave_merge128_desc(acc, b[i]);
  }
#pragma unroll
  for (int st = 1; st < NW; st <<= 1) {
    if ((w & (2 * st - 1)) == st) {
      tree[w][l] = acc[0];
      tree[w][kWave + l] = acc[1];
    }
    __syncthreads();
    if ((w & (2 * st - 1)) == 0 && w + st < a.nseg) {  // waves from nseg on hold no list
      const uint64_t c[2] = {tree[w + st][l], tree[w + st][kWave + l]};
      wave_merge128_desc(acc, c);
    }
  }
  if (w == 0) {
    tree[0][l] = acc[0];
    tree[0][kWave + l] = acc[1];
  }
  __syncthreads();
  if (!SAMPLE && a.lists_only) {  // the row's merged list (already in the shard's column frame)
    for (int i = threadIdx.x; i < kRun; i += kMergeNT) a.out_lists[(size_t)row * kRun + i] = tree[0][i];
    return;
  }
  finalize_row<DT, SAMPLE>(a, row, tree[0], sg, rp);
}

// Kernel B for top-k with k <= 64 (no sampler, no lists out): the first 64
// entries of each segment's sorted list hold the segment's part of the row's
// top-k, so the lists are merged as 64-entry runs (one entry per lane, half
// the merge network of the 128-entry runs).
template <int DT>
__global__ __launch_bounds__(kMergeNT) void seg_merge64_kernel(SelArgs a) {
  constexpr int NW = kMergeNT / kWave;
  constexpr int PER = kMaxSeg / NW;  // lists per wave, at most
  __shared__ uint64_t tree[NW][kWave];
  __shared__ float sg[kRun];
  const int64_t row = blockIdx.x;
  const int w = threadIdx.x / kWave, l = lane_id();
  const uint64_t* src = a.ws_lists + (size_t)row * a.nseg * kRun;
  const RowParams rp = load_row_params<false>(a, row);
  uint64_t b[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int sgi = w + i * NW;
    b[i] = sgi < a.nseg ? src[sgi * kRun + l] : 0ull;
  }
  uint64_t acc = b[0];
#pragma unroll
  for (int i = 1; i < PER; ++i) {
    if (w + i * NW < a.nseg) acc = wave_merge64_desc(acc, b[i]);
  }
#pragma unroll
  for (int st = 1; st < NW; st <<= 1) {
    if ((w & (2 * st - 1)) == st) tree[w][l] = acc;
    __syncthreads();
    if ((w & (2 * st - 1)) == 0 && w + st < a.nseg) acc = wave_merge64_desc(acc, tree[w + st][l]);
  }
  if (w == 0) tree[0][l] = acc;
  __syncthreads();
  finalize_row<DT, false>(a, row, tree[0], sg, rp);  // reads the first k <= 64 entries
}

// Kernel B for top-k with k <= 64 over at most two lists per row (the
// whole-row kernel's two parts): one wave per row merges the two 64-entry
// runs in registers and writes the outputs, no LDS tree and no barrier.
template <int DT>
__global__ __launch_bounds__(kWave) void seg_merge64_pair_kernel(SelArgs a) {
  __shared__ uint64_t list[kWave];
  __shared__ float sg[kRun];
  const int64_t row = blockIdx.x;
  const int l = lane_id();
  const uint64_t* src = a.ws_lists + (size_t)row * a.nseg * kRun;
  const RowParams rp = load_row_params<false>(a, row);
  uint64_t acc = src[l];
  if (a.nseg > 1) acc = wave_merge64_desc(acc, src[kRun + l]);
  list[l] = acc;
  __syncthreads();
  finalize_row<DT, false>(a, row, list, sg, rp);  // reads the first k <= 64 entries
}

// ---------------------------------------------------------------------------
// Kernel S (stream_select_kernel): a whole row (or one equal part of it) per
// 1024-thread workgroup (16 waves, 4 per SIMD), V 16-byte vectors per thread
// (V <= 19), vector j of thread t at row vector j * 1024 + t.
//   1. Every load is issued up front.
//   2. The bound L: the minimum over waves 0..7 of each one's 16th largest
//      thread maximum (8th when only 64 list places are read), a radix search
//      with one ballot per key bit, so at least 128 (64) elements reach L.
//      Those waves' loads are issued first and
//      arrive first, so L is known before waves 8..15 have their first
//      vector (measured at config 4: 16.86 -> 16.15 us against the bound over
//      all 16 waves; waves 0..11 gave 17.0 us, waves 0..3 overflow the
//      candidate array).
//   3. Vectors whose maximum reaches L are staged in their wave's LDS region
//      (one ballot per vector index; waves 8..15 stage each vector as it
//      arrives, at raised wave priority), then each wave takes its staged
//      vectors one per lane and
//      appends the elements >= L as composites (canonical key << 32 |
//      ~index).  The row maximum M the rank needs is at least the largest
//      candidate key: waves 0..7 post their largest element, waves 8..15
//      their largest candidate.
//   4. The candidates are put in order by an LDS bucket rank: buckets of
//      (M - key) >> shift (at most kBuckets), one atomic per candidate for the
//      histogram and its slot, an exclusive scan, a scatter, and each
//      candidate's rank = its bucket's start + the larger composites in its
//      bucket.  The first 128 (64) ranks are the row's top-128 (64) in order.
// Rows with fewer than 128 eligible elements rank them and take the rest of
// the list by class (fill_ineligible).  Rows whose staged vectors or
// candidates overflow (heavy ties: constant rows, long tie blocks) take
// tie_select over the whole row instead (stream_tie_path).  Both rare paths
// are out of line: the kernel's hot code is 31 KB instead of 50 KB (measured
// at config 4 together with step 3's per-vector staging: 16.2 -> 15.8 us).
// ---------------------------------------------------------------------------
constexpr int kNTS = 1024;
constexpr int kStageCap = 128;   // staged vectors per wave
constexpr int kCandCap = 1024;   // candidates (one per thread in the ranking)
constexpr int kBuckets = 1024;

struct StreamShared {
  uint4 vst[kNTS / kWave][kStageCap];      // staged vectors, per wave     32 KiB
  uint32_t vsi[kNTS / kWave][kStageCap];   // their first element's row index
  uint64_t cand[kCandCap + 8];             // candidates, then in bucket order (+8: unguarded reads)
  int hist[kBuckets];                      // bucket counts, then bucket starts
  uint32_t wl[kNTS / kWave];
  uint32_t wm[kNTS / kWave];
  uint32_t posted;  // bit w: wave w (< 8) has its bound term in wl
  int ncand;
  int ovf;                                 // a wave's staged vectors overflowed its region
};

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4_t* GlobalVec;

// Loaded in place of vectors past the end of a row: all-ones (negative NaNs)
// never pass a filter and never raise a maximum.
static __device__ u32x4_t g_dead_vec = {~0u, ~0u, ~0u, ~0u};

// lanes below this one in the wave
__device__ __forceinline__ uint64_t lanes_below() {
  const int l = lane_id();
  return l == 0 ? 0ull : (~0ull >> (kWave - l));
}

// The k-th largest (kth) and the largest (top) of the wave's 64 values
// (k >= 1), by radix searches over the bits with one ballot per bit and
// search: the largest K with #(v >= K) >= k.
template <int BITS>
__device__ __forceinline__ void wave_kth_and_max(uint32_t v, int k, uint32_t& kth, uint32_t& top) {
  uint32_t K = 0, T = 0;
#pragma unroll
  for (int b = BITS - 1; b >= 0; --b) {
    const uint32_t pk = K | (1u << b), pt = T | (1u << b);
    const uint64_t mk = __ballot(v >= pk), mt = __ballot(v >= pt);
    K = __popcll(mk) >= k ? pk : K;
    T = mt ? pt : T;
  }
  kth = K;
  top = T;
}


// Slots q < lo or q >= hi of a 16-byte vector of VEC elements become all-ones.
template <int DT>
__device__ __forceinline__ uint4 kill_slots(uint4 x, int lo, int hi) {
  constexpr int VEC = ElemT<DT>::VEC;
  uint32_t d[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int q = 0; q < VEC; ++q) {
    const bool dead = q < lo || q >= hi;
    if (DT == kBF16) d[q >> 1] |= dead ? ((q & 1) ? 0xFFFF0000u : 0x0000FFFFu) : 0u;
    else d[q] |= dead ? ~0u : 0u;
  }
  return make_uint4(d[0], d[1], d[2], d[3]);
}

// Bits q of the elements of vv with canonical key >= thr (thr >= the smallest
// eligible key, so NaNs and dead slots never pass).
template <int DT>
__device__ __forceinline__ uint32_t pass_mask_ge(const uint4 vv, uint32_t thr) {
  constexpr bool kBF = DT == kBF16;
  constexpr int VEC = ElemT<DT>::VEC;
  constexpr uint32_t kZeroKey = kBF ? 0x8000u : 0x80000000u;
  constexpr int32_t kPosInf = kBF ? 0x7F80 : 0x7F800000;
  uint32_t m = 0;
  if (thr > kZeroKey) {  // positive threshold: st <= bits <= +inf in the signed view
    const int32_t st = (int32_t)(thr - kZeroKey);
    const uint32_t span = (uint32_t)(kPosInf - st);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t x = dword_of(vv, d);
      if (kBF) {
        m |= ((uint32_t)((int32_t)(int16_t)(x & 0xFFFFu) - st) <= span ? 1u : 0u) << (2 * d);
        m |= ((uint32_t)(((int32_t)x >> 16) - st) <= span ? 1u : 0u) << (2 * d + 1);
      } else {
        m |= ((uint32_t)((int32_t)x - st) <= span ? 1u : 0u) << d;
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < VEC; ++q) m |= (Sel<DT, true>::canon(elem_bits<DT>(vv, q)) >= thr ? 1u : 0u) << q;
  }
  return m;
}

// Class masks of a 16-byte vector for the ineligible classes: finfo.min
// elements in bits 0-7, -inf in bits 8-15, NaN in bits 16-23 (all slots,
// dead ones included).
template <int DT>
__device__ __forceinline__ uint32_t ineligible_masks(const uint4 v) {
  constexpr bool kBF = DT == kBF16;
  constexpr int VEC = ElemT<DT>::VEC;
  constexpr uint32_t kMinB = kBF ? 0xFF7Fu : 0xFF7FFFFFu, kNegInfB = kBF ? 0xFF80u : 0xFF800000u;
  constexpr uint32_t kAbs = kBF ? 0x7FFFu : 0x7FFFFFFFu, kInfAbs = kBF ? 0x7F80u : 0x7F800000u;
  uint32_t m = 0;
#pragma unroll
  for (int q = 0; q < VEC; ++q) {
    const uint32_t b = elem_bits<DT>(v, q);
    m |= (b == kMinB ? 1u : 0u) << q;
    m |= (b == kNegInfB ? 1u : 0u) << (8 + q);
    m |= ((b & kAbs) > kInfAbs ? 1u : 0u) << (16 + q);
  }
  return m;
}

// The smallest (bits - finfo.min's bits) over the elements of a 16-byte
// vector, wrapping in the element width: 0 when the vector holds finfo.min,
// 1 when it holds -inf but not finfo.min, larger otherwise.
template <int DT>
__device__ __forceinline__ uint32_t min_offset_from_min(const uint4 v) {
  if (DT == kBF16) {
    const ushort2_t fm = __builtin_bit_cast(ushort2_t, 0xFF7FFF7Fu);
    ushort2_t m = __builtin_bit_cast(ushort2_t, v.x) - fm;
    m = __builtin_elementwise_min(m, __builtin_bit_cast(ushort2_t, v.y) - fm);
    m = __builtin_elementwise_min(m, __builtin_bit_cast(ushort2_t, v.z) - fm);
    m = __builtin_elementwise_min(m, __builtin_bit_cast(ushort2_t, v.w) - fm);
    const uint32_t mm = __builtin_bit_cast(uint32_t, m);
    const uint32_t lo = mm & 0xFFFFu, hi = mm >> 16;
    return lo < hi ? lo : hi;
  }
  const uint32_t a = v.x - 0xFF7FFFFFu, b = v.y - 0xFF7FFFFFu, c = v.z - 0xFF7FFFFFu, d = v.w - 0xFF7FFFFFu;
  const uint32_t ab = a < b ? a : b, cd = c < d ? c : d;
  return ab < cd ? ab : cd;
}

// Rows with fewer than 128 eligible elements, all n of them candidates:
// list[n..127] <- the first 128 - n ineligible elements in composite order --
// the finfo.min elements, then -inf, then NaN, each class in index order --
// and zeros where the row has fewer than 128 elements.  pmin / pinf: this
// thread's vectors j (bit j) that may hold finfo.min or -inf, from the first
// read (NaNs are not tracked: every vector may hold one); the vectors that
// hold a class anywhere in the row are read again one at a time (vector j of
// thread t at row vector j * kNTS + t of the aligned base, nv vectors, the
// row's first element at slot mis), in order, until the list is full.
// tmp: 2 * 16 words of LDS.  Out of line: a rare path kept out of the
// kernel's hot code (the kernel's code size sets its instruction-cache
// footprint).
template <int DT, int V>
__device__ __attribute__((noinline)) void fill_ineligible(const uint4* row_base, int nv, int mis, int cols, int n,
                                                          uint32_t pmin, uint32_t pinf, uint64_t* list, int* red,
                                                          uint32_t* tmp) {
  constexpr bool kBF = DT == kBF16;
  constexpr int VEC = ElemT<DT>::VEC, NW = kNTS / kWave;
  constexpr uint32_t kMinKey = kBF ? 0x0080FFFFu : 0x00800000u;  // global keys of the three classes
  constexpr uint32_t kNegInfKey = 0x007FFFFFu, kNaNKey = 1u;
  const int tid = threadIdx.x;
  const int w = tid / kWave, l = lane_id();
  const GlobalVec gb = (GlobalVec)row_base;
  const GlobalVec dead = (GlobalVec)(uintptr_t)&g_dead_vec;
  pmin = wave_or_u32(pmin);
  pinf = wave_or_u32(pinf);
  if (l == 0) {
    tmp[w] = pmin;
    tmp[NW + w] = pinf;
  }
  __syncthreads();
  pmin = 0;
  pinf = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    pmin |= tmp[i];
    pinf |= tmp[NW + i];
  }
  constexpr uint32_t kAll = (1u << V) - 1u;
  int r = kMaxK - n, base = n;
#pragma unroll 1
  for (int c = 0; c < 3 && r > 0; ++c) {  // block-uniform
    uint32_t pres = c == 0 ? pmin : (c == 1 ? pinf : kAll);
    const uint32_t key = c == 0 ? kMinKey : (c == 1 ? kNegInfKey : kNaNKey);
    while (pres && r > 0) {  // block-uniform: the vectors that may hold the class, in order
      const int j = __builtin_ctz(pres);
      pres &= pres - 1u;
      const int v = j * kNTS + tid;
      const u32x4_t x = *(v < nv ? gb + v : dead);
      const int e0 = v * VEC - mis;
      uint32_t m = (ineligible_masks<DT>(make_uint4(x.x, x.y, x.z, x.w)) >> (8 * c)) & 0xFFu;
#pragma unroll
      for (int q = 0; q < VEC; ++q)  // slots outside the row
        m &= (uint32_t)(e0 + q) < (uint32_t)cols ? ~0u : ~(1u << q);
      int total;
      int p = block_exscan<NW>(__popc(m), red, total);
      while (m && p < r) {
        const int q = __builtin_ctz(m);
        m &= m - 1u;
        list[base + p] = make_comp(key, (uint32_t)(e0 + q));
        ++p;
      }
      const int took = total < r ? total : r;
      base += took;
      r -= took;
    }
  }
  for (int i = base + tid; i < kMaxK; i += kNTS) list[i] = 0ull;
}

// Rows whose staged vectors or candidates overflow (heavy ties): tie_select
// over the whole row, then the block's merge, into the sorted 128-entry list.
// Out of line, like fill_ineligible.
template <int DT, int V>
__device__ __attribute__((noinline)) void stream_tie_path(
    const uint4* base, int nv, int mis, int cols,
    SegShared<typename Sel<DT, (kNTS * V * ElemT<DT>::VEC > 65535)>::Comp, kNTS>& sh, uint4* stage) {
  using ST = Sel<DT, (kNTS * V * ElemT<DT>::VEC > 65535)>;
  constexpr int VEC = ElemT<DT>::VEC;
  const int tid = threadIdx.x, w = tid / kWave, l = lane_id();
  const int lbase = tid * VEC;
  const int64_t seg_e0 = -(int64_t)mis;
  const int live_lo = mis;
  const int live_hi = cols + mis < nv * VEC ? cols + mis : nv * VEC;
  const int wcnt = tie_select<DT, V, kNTS, 2>(base, 0, nv, lbase, live_lo, live_hi, (uint32_t)seg_e0, kMaxK,
                                              sh.cand + w * Geo<kNTS>::WCAP, sh.red, stage);
  if (l == 0) sh.wc[w] = wcnt;
  __syncthreads();
  block_select(sh, (const int*)sh.wc);
  for (int i = tid; i < kRun; i += kNTS) sh.list64[i] = ST::to_global(sh.list[i], seg_e0);
}

template <int DT, int V, bool SAMPLE, bool EDGE>
__global__ __launch_bounds__(kNTS) void stream_select_kernel(SelArgs a) {
  using T = ElemT<DT>;
  constexpr int VEC = T::VEC, ES = T::ES, NW = kNTS / kWave;
  static_assert(V <= 31, "one bit per vector in 32-bit masks");
  constexpr bool kBF = DT == kBF16;
  constexpr int KB = kBF ? 16 : 32;  // canonical key bits
  using ST = Sel<DT, (kNTS * V * VEC > 65535)>;  // the tie path's composites (tie_select's choice)
  using CT = typename ST::Comp;
  constexpr uint32_t kZeroKey = kBF ? 0x8000u : 0x80000000u;
  constexpr int32_t kPosInf = kBF ? 0x7F80 : 0x7F800000;
  constexpr int32_t kOrdNegInf = kBF ? -32641 : (int32_t)0x807FFFFFu;
  constexpr uint32_t kFloor = kBF ? 0x0081u : 0x00800001u;  // smallest eligible canonical key
  __shared__ StreamShared ss;
  __shared__ SegShared<CT, kNTS> sh;  // tie path, output list
  __shared__ uint4 stage[2 * kNTS];   // tie path
  const int tid = threadIdx.x, w = tid / kWave, l = lane_id();
  const int64_t row = blockIdx.x;
  const char* rowp = (const char*)a.x + (size_t)(row * a.cols) * ES;
  const RowVec<ES> rv(rowp);
  const int nv = (int)((a.cols + rv.mis + VEC - 1) / VEC);  // 1 <= nv <= kNTS * V (host plan)
  // list places the consumer reads: the bound guarantees kq elements, the
  // rank writes places below kq (the rest of the list is not read)
  const int kq = a.list_k == 64 ? 64 : kMaxK;
  const int cols = (int)a.cols;
  const RowParams rp = load_row_params<SAMPLE>(a, row);

  if (tid == 0) ss.posted = 0;
  lds_barrier();  // posted is clear before any wave posts; no load is in flight yet

  // ---- 1. every load up front (global loads: flat loads would also count
  // against the LDS counter)
  uint4 raw[V];
  {
    const GlobalVec gb = (GlobalVec)rv.base;
    const GlobalVec dead = (GlobalVec)(uintptr_t)&g_dead_vec;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int v = j * kNTS + tid;
      const u32x4_t x = __builtin_nontemporal_load(v < nv ? gb + v : dead);
      raw[j] = make_uint4(x.x, x.y, x.z, x.w);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // every load issues before any use of one
  if (tid == 0) {
    ss.ncand = 0;
    ss.ovf = 0;
  }
  for (int i = tid; i < kBuckets; i += kNTS) ss.hist[i] = 0;
  // The row's first vector (misaligned start, thread 0, j = 0) and last one
  // (partial end) hold slots outside the row, only when EDGE (the host
  // launches the EDGE = false kernel when every row starts 16-byte aligned
  // and cols is a multiple of the vector width).  Their outside slots become
  // all-ones, under block-uniform conditions and with selects of values
  // only (a store guarded per vector would be merged into a store at a
  // variable index, which would move raw[] to scratch memory).  One thread
  // may own both, as different vectors.
  if (EDGE) {
    const int tail_live = cols + rv.mis - (nv - 1) * VEC;  // live slots of the last vector, 1..VEC
    if (rv.mis > 0 || tail_live < VEC) {
      int hj = -1, tj = -1, lo = 0, hi = VEC;
      if (tid == 0 && rv.mis > 0) {
        hj = 0;
        lo = rv.mis;
      }
      if (tid == (nv - 1) % kNTS && tail_live < VEC) {
        tj = (nv - 1) / kNTS;
        hi = tail_live;
      }
      // the empty asm keeps the masks derived from these values in this block
      asm volatile("" : "+v"(hj), "+v"(tj), "+v"(lo), "+v"(hi));
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const uint4 x = raw[j];
        const uint4 y = kill_slots<DT>(x, hj == j ? lo : 0, tj == j ? hi : VEC);
        const bool t = hj == j || tj == j;
        raw[j] = make_uint4(t ? y.x : x.x, t ? y.y : x.y, t ? y.z : x.z, t ? y.w : x.w);
      }
    }
  }

  // staging: vectors j with flag f go to the wave's own LDS region, one per
  // slot in lane order; wcnt counts them (past kStageCap: ovf)
  int wcnt = 0;
  auto stage_if = [&](int j, bool f) {
    const uint64_t m = __ballot(f);
    if (m) {
      if (f) {
        const int o = wcnt + (int)__popcll(m & lanes_below());
        if (o < kStageCap) {
          ss.vst[w][o] = raw[j];
          ss.vsi[w][o] = (uint32_t)((j * kNTS + tid) * VEC - rv.mis);
        }
      }
      wcnt += (int)__popcll(m);
    }
  };
  // the wave's staged vectors, one per lane: elements with key >= thr are
  // appended to the candidates; post_top: the wave's M term is the largest
  // key it appended
  auto extract = [&](uint32_t thr, bool post_top) {
    if (l == 0 && wcnt > kStageCap) ss.ovf = 1;
    const int nst = wcnt < kStageCap ? wcnt : kStageCap;
    uint32_t top = 0;  // the largest key appended by this lane
    for (int r0 = 0; r0 < nst; r0 += kWave) {  // wave-uniform
      const int o = r0 + l;
      uint32_t pm = 0;
      uint4 vv = make_uint4(~0u, ~0u, ~0u, ~0u);
      uint32_t e0 = 0;
      if (o < nst) {
        vv = ss.vst[w][o];
        e0 = ss.vsi[w][o];
        pm = pass_mask_ge<DT>(vv, thr);
      }
      int tot;
      const int pre = wave_exscan_i32(__popc(pm), tot);
      if (tot) {
        int b0 = 0;
        if (l == 0) b0 = atomicAdd(&ss.ncand, tot);
        int oc = __shfl(b0, 0) + pre;
        while (pm) {
          const int q = __builtin_ctz(pm);
          pm &= pm - 1u;
          const uint32_t kk = Sel<DT, true>::canon(elem_bits<DT>(vv, q));
          top = kk > top ? kk : top;
          if (oc < kCandCap) ss.cand[oc] = make_comp(kk, e0 + (uint32_t)q);
          ++oc;
        }
      }
    }
    if (post_top) {
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) {
        const uint32_t o = lane_xor(top, d);
        top = o > top ? o : top;
      }
      if (l == 0) ss.wm[w] = top;
    }
  };

  uint32_t thr, M;
  uint32_t pmin = 0, pinf = 0;  // rows with thr at the floor: the vectors that may hold finfo.min / -inf
  // ---- 2. the bound L from waves 0..7 alone: the minimum over them of each
  // one's 16th largest thread maximum, so at least 128 elements of the row
  // reach it.  Their loads are issued first and arrive first, so L is posted
  // before waves 8..15 have their first vector, and those stage each vector
  // as it arrives.
  constexpr int NE = NW / 2;
  const bool early = w < NE;
  int32_t vmax[V];  // early waves: their vectors' maxima, kept for the staging
  {
    if (early) {
#pragma unroll
      for (int j = 0; j < V; ++j) vmax[j] = vec_smax<DT>(raw[j]);
      int32_t smax = vmax[0];
#pragma unroll
      for (int j = 1; j < V; ++j) smax = imax32(smax, vmax[j]);
      uint32_t tk;  // canonical key of the thread's largest element
      if (smax >= 0 && smax <= kPosInf) {
        tk = (uint32_t)smax | kZeroKey;
      } else {
        int32_t omax = kBF ? -32768 : (int32_t)0x80000000u;
#pragma unroll
        for (int j = 0; j < V; ++j) omax = imax32(omax, vec_omax<DT>(raw[j]));
        if (omax <= kPosInf) {
          tk = omax < kOrdNegInf ? 0u : (omax == -1 ? kZeroKey : (uint32_t)omax + kZeroKey);
        } else {  // a positive NaN: canonical maximum element by element
          tk = 0;
#pragma unroll
          for (int j = 0; j < V; ++j) {
#pragma unroll
            for (int q = 0; q < VEC; ++q) {
              const uint32_t kk = Sel<DT, true>::canon(elem_bits<DT>(raw[j], q));
              tk = kk > tk ? kk : tk;
            }
          }
        }
      }
      uint32_t wl, wm;
      wave_kth_and_max<KB>(tk, kq / NE, wl, wm);
      if (l == 0) {
        ss.wl[w] = wl;
        ss.wm[w] = wm;
        __hip_atomic_fetch_or(&ss.posted, 1u << w, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
    while ((__hip_atomic_load(&ss.posted, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) & ((1u << NE) - 1u)) !=
           ((1u << NE) - 1u))
      __builtin_amdgcn_s_sleep(1);
    uint32_t L = ss.wl[0];
#pragma unroll
    for (int i = 1; i < NE; ++i) L = ss.wl[i] < L ? ss.wl[i] : L;
    thr = L > kFloor ? L : kFloor;

    // ---- 3. stage the vectors that may hold a candidate (each as soon as it
    // is in: the wait for vector j sits before its maximum), then the
    // candidates
    const bool pos_thr = thr > kZeroKey;
    const int32_t st = (int32_t)(thr - kZeroKey);                       // bits, positive threshold
    const int32_t ot = thr == kZeroKey ? -1 : (int32_t)(thr - kZeroKey);  // ordered view otherwise
    // Two ifs, not if/else (the empty asm keeps the compiler from merging
    // them): the join of an if/else leaves the other side's values undefined,
    // and the code generator reads such an undefined register with a wait for
    // every load in flight.
    if (pos_thr) {  // block-uniform: the signed-view maxima decide
      if (early) {
#pragma unroll
        for (int j = 0; j < V; ++j) stage_if(j, vmax[j] >= st);
      } else {
        // the late waves' staging and extraction are the critical path: they
        // issue ahead of the early waves' extraction on the shared SIMDs
        // (config 4: 15.78 -> 15.44 us; priority 3, or also raising the
        // early waves for their bound, no better)
        __builtin_amdgcn_s_setprio(2);
#pragma unroll
        for (int j = 0; j < V; ++j) stage_if(j, vec_smax<DT>(raw[j]) >= st);
      }
    }
    uint32_t thr_b = __builtin_amdgcn_readfirstlane(thr);
    asm volatile("" : "+s"(thr_b));
    if (thr_b <= kZeroKey) {
#pragma unroll
      for (int j = 0; j < V; ++j) stage_if(j, vec_omax<DT>(raw[j]) >= ot);
      if (thr == kFloor) {  // block-uniform: the row may hold fewer than 128 eligible elements
        // vectors that hold finfo.min, and those that may hold -inf (cheap
        // packed tests; NaNs are not tracked: every vector may hold one)
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const uint32_t o = min_offset_from_min<DT>(raw[j]);
          pmin |= (o == 0u ? 1u : 0u) << j;
          pinf |= (o <= 1u ? 1u : 0u) << j;
        }
      }
    }
    extract(thr, !early);
    __builtin_amdgcn_s_setprio(0);
  }
  __syncthreads();
  // M: at least the largest candidate key (waves 0..7 post their largest
  // element, waves 8..15 their largest candidate), all the rank needs
  M = ss.wm[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) M = ss.wm[i] > M ? ss.wm[i] : M;
  const int n = ss.ncand;
  // fewer than 128 with thr at the eligibility floor: every eligible element
  // of the row is a candidate, the rest of the list is ineligible elements
  const bool fill = ss.ovf == 0 && n < kq && thr == kFloor;  // block-uniform
  // an overflowing staging region or more than kCandCap candidates: heavy ties
  const bool tie = !fill && (ss.ovf != 0 || n < kq || n > kCandCap);
  if (fill) fill_ineligible<DT, V>(rv.base, nv, rv.mis, cols, n, pmin, pinf, sh.list64, sh.red, &ss.vsi[0][0]);
  if (tie) {
    stream_tie_path<DT, V>(rv.base, nv, rv.mis, cols, sh, stage);
  } else if (n > 0) {
    // ---- 4. bucket rank
    const uint32_t range = M - thr;  // the candidates' keys lie in [thr, M]
    int shift = 0;
    while ((range >> shift) >= (uint32_t)kBuckets) ++shift;
    const bool mine = tid < n;
    const uint64_t c = mine ? ss.cand[tid] : 0ull;
    const int b = mine ? (int)((M - comp_key(c)) >> shift) : 0;
    int slot = 0;
    if (mine) slot = atomicAdd(&ss.hist[b], 1);
    __syncthreads();
    const int nb = (int)(range >> shift) + 1;
    if (w == 0) {  // exclusive scan of the bucket counts, 16 buckets per lane
      constexpr int PER = kBuckets / kWave;
      int cnt[PER];
      int loc = 0;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        cnt[i] = ss.hist[l * PER + i];  // buckets past nb hold 0
        loc += cnt[i];
      }
      int tot;
      int run = wave_exscan_i32(loc, tot);
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        ss.hist[l * PER + i] = run;  // the bucket's start
        run += cnt[i];
      }
    }
    __syncthreads();
    // buckets that start at rank >= 128 are not needed any further
    int start = 0, end = 0;
    const bool need = mine && (start = ss.hist[b]) < kq;
    if (need) {
      end = b + 1 < nb ? ss.hist[b + 1] : n;
      ss.cand[start + slot] = c;  // every thread read its own entry before the barriers above
    }
    __syncthreads();
    if (need) {
      int r = start;
      for (int i0 = start; i0 < end; i0 += 8) {  // 8 LDS reads in flight (unguarded: the array is padded)
        uint64_t x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = ss.cand[i0 + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) r += (i0 + u < end && x[u] > c) ? 1 : 0;
      }
      if (r < kq) {
        const uint32_t k = comp_key(c);
        uint32_t key = k;
        if (kBF) key = k >= 0x8000u ? (k << 16) : ((k << 16) | 0xFFFFu);
        sh.list64[r] = make_comp(key, ~(uint32_t)c);
      }
    }
  }
  __syncthreads();
  if (!a.lists_only) {
    finalize_row<DT, SAMPLE>(a, row, sh.list64, sh.samp_g, rp);
  } else {
    uint64_t* dst = a.ws_lists + (size_t)row * kRun;
    const uint64_t off = (uint64_t)(a.col_offset + (a.nparts > 1 ? (row % a.nparts) * a.part_cols : 0));
    for (int i = tid; i < kq; i += kNTS) dst[i] = sh.list64[i] ? sh.list64[i] - off : 0ull;
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
  float v[2], e[2], g[2];
  int32_t id[2];
  const float v0 = __uint_as_float(T::load_bits(rowp, 0));
  const uint32_t row_ctr = (uint32_t)(row + dim0_offset);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int p = h * kWave + l;
    v[h] = p < K ? __uint_as_float(T::load_bits(rowp, p)) : 0.0f;
    id[h] = p < K ? idx[row * K + p] : 0;
    e[h] = p < K ? candidate_exp(v[h], v0) : 0.0f;
    g[h] = p < K ? candidate_noise(rng_key[0], rng_key[1], row_ctr, vocab, id[h]) : 0.0f;
  }
  const float thr = top_p_threshold(v, e, K, top_p[row]);
  const int32_t tok = gumbel_argmax(v, id, g, K, thr, temperature[row], replace_f32);
  if (l == 0) out[row] = tok;
}

// Standalone top_p_mask (sampling.py:25-62), axis 0: f32 candidates
// [K, cols] sorted descending down each column, K <= 128; one wave per column
// (position p = h * 64 + lane).  Keeps v >= the threshold of top_p_threshold,
// writes replace_f32 elsewhere.
__global__ __launch_bounds__(kWave) void top_p_mask_kernel(const float* logits, int64_t cols, int K,
                                                           const float* top_p, float replace_f32, float* out) {
  const int64_t b = blockIdx.x;
  const int l = lane_id();
  float v[2], e[2];
  const float v0 = logits[b];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int p = h * kWave + l;
    v[h] = p < K ? logits[(int64_t)p * cols + b] : 0.0f;
    e[h] = p < K ? candidate_exp(v[h], v0) : 0.0f;
  }
  const float thr = top_p_threshold(v, e, K, top_p[b]);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int p = h * kWave + l;
    if (p < K) out[(int64_t)p * cols + b] = v[h] >= thr ? v[h] : replace_f32;
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct Plan {
  int nt;  // threads per workgroup: kNT (segments) or kNTS (whole rows)
  int maxv;
  int nseg;
  int64_t vps;
  int parts;  // > 1: whole-row kernel on that many equal parts of each row, then the merge
};

// Work split.  A row of nv 16-byte vectors is handled either
//   * whole by one 1024-thread workgroup of stream_select_kernel (up to 19
//     vectors per thread) whenever the row fits: no merge kernel at all.  At
//     small row counts one workgroup per row leaves most CUs idle, but a
//     256 KiB row streams into one workgroup in ~6 us (at most ~40 GB/s),
//     less than the segment path's bound-after-loads plus second launch
//     (measured, A/B: sampler [1, 128256] bf16 13.0 -> 9.0 us, [64, 128256]
//     16.6 -> 11.7; top-k [8, 32768] f32 9.90 -> 8.05, [100, 65472] f32
//     16.7 -> 11.8; 19 vectors per thread for the 151936-wide bf16
//     vocabulary: sampler [64, 151936] 20.5 -> 12.7, [256, 151936] 25.2 ->
//     17.8; no shape slower); or
//   * as 2-4 equal parts of at most 19 vectors per thread when the row
//     divides and rows x parts <= kPartsMaxBlocks: the whole-row kernel
//     writes each part's top-128 list (rows of the [parts x rows, cols /
//     parts] view, column offsets added back), then the per-row merge
//     (config 3, [128, 151936] f32: 21.50 -> 20.05 us; f32 sampler
//     [64, 128256] 19.5 -> 15.7, [64, 201088] 26.9 -> 17.2; at more blocks
//     the segments win: [256, 201088] 46.5 against 50.4, [512, 151936]
//     top-k 55.1 against 62.6); or
//   * in segments of 256 x MAXV vectors, MAXV in {4, 8, 16, 19}: the largest that
//     still gives ~4 workgroups per CU over the launch, then a per-row merge;
//     where 16 gives more than one residency round (4 workgroups per CU,
//     kTargetBlocks) and 19 gives exactly one, MAXV = 19 (config 3: 8
//     segments of 19 vectors per thread instead of 10 of 16, measured
//     22.03 -> 21.45 us).
static int plan_rows(int64_t rows, int64_t cols, int dt, Plan* p) {
  const int vec = dt == kF32 ? 4 : 8;
  const int64_t nv = (cols + 2 * (vec - 1)) / vec;  // covers any row misalignment
  static const int kOpts[3] = {16, 8, 4};
  p->parts = 0;
  if (nv <= (int64_t)kNTS * 19) {
    int maxv = nv > (int64_t)kNTS * 16 ? 19 : 16;
    while (maxv > 4 && (int64_t)kNTS * (maxv / 2) >= nv) maxv /= 2;
    p->nt = kNTS;
    p->maxv = maxv;
    p->nseg = 1;
    p->vps = (int64_t)kNTS * maxv;
    return kOk;
  }
  for (int np = 2; np <= 4 && rows * np <= kPartsMaxBlocks; ++np) {  // equal whole-row parts
    if (cols % np) continue;
    const int64_t nvh = (cols / np + 2 * (vec - 1)) / vec;
    if (nvh <= (int64_t)kNTS * 19) {
      p->nt = kNTS;
      p->maxv = nvh > (int64_t)kNTS * 16 ? 19 : 16;
      p->nseg = np;
      p->vps = (int64_t)kNTS * p->maxv;
      p->parts = np;
      return kOk;
    }
  }
  int maxv = 4;
  for (int o = 0; o < 3; ++o) {
    const int64_t per = (int64_t)kNT * kOpts[o];
    const int64_t nseg = (nv + per - 1) / per;
    if (rows * nseg >= kTargetBlocks && nseg <= kMaxSeg) { maxv = kOpts[o]; break; }
  }
  int64_t per = (int64_t)kNT * maxv;
  int64_t nseg = (nv + per - 1) / per;
  if (maxv == 16 && rows * nseg > kTargetBlocks) {  // one residency round with 19 vectors per thread?
    const int64_t per19 = (int64_t)kNT * 19;
    const int64_t nseg19 = (nv + per19 - 1) / per19;
    if (rows * nseg19 <= kTargetBlocks && nseg19 >= 2 && nseg19 <= kMaxSeg) {
      p->nt = kNT;
      p->maxv = 19;
      p->nseg = (int)nseg19;
      p->vps = per19;
      return kOk;
    }
  }
  while (nseg > kMaxSeg && maxv < 16) {
    maxv *= 2;
    per = (int64_t)kNT * maxv;
    nseg = (nv + per - 1) / per;
  }
  if (nseg > kMaxSeg) {
    set_error("row length %lld exceeds this build's limit of %d segments", (long long)cols, kMaxSeg);
    return kUnsupported;
  }
  p->nt = kNT;
  p->maxv = maxv;
  p->nseg = (int)nseg;
  p->vps = per;
  return kOk;
}

static size_t ws_bytes_for(int64_t rows, const Plan& p) {
  if (p.nseg <= 1) return 0;
  return (size_t)rows * p.nseg * kRun * sizeof(uint64_t);
}

template <int DT, int MAXV, int NT, bool SAMPLE>
static void launch_a(const SelArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((seg_select_kernel<DT, MAXV, NT, SAMPLE>), dim3((unsigned)(a.nseg * a.rows)), dim3(NT), 0, s,
                     a);
}

template <int DT, bool SAMPLE>
static int launch_select(const SelArgs& a0, const Plan& p, hipStream_t s, const char* what) {
  // parts: the whole-row kernel writes each part's list (no sampling; its
  // rows are the [np rows, cols / np] view), the merge kernel finishes the row
  SelArgs h = a0;
  // top-k with k <= 64 reads the first 64 places of a row's (or a part's) list
  if (!SAMPLE && !a0.lists_only && a0.k <= kWave) h.list_k = kWave;
  if (p.parts > 1) {
    h.rows = a0.rows * p.parts;
    h.cols = a0.cols / p.parts;
    h.nseg = 1;
    h.lists_only = 1;
    h.part_cols = h.cols;
    h.nparts = p.parts;

  }
  const SelArgs& a = h;
  if (p.nt == kNTS && p.parts > 1) {
    const bool edge = ((uintptr_t)a.x % 16) != 0 || (a.cols * ElemT<DT>::ES) % 16 != 0;
    const dim3 g((unsigned)a.rows), b(kNTS);
    if (p.maxv == 19) {
      if (edge) hipLaunchKernelGGL((stream_select_kernel<DT, 19, false, true>), g, b, 0, s, a);
      else hipLaunchKernelGGL((stream_select_kernel<DT, 19, false, false>), g, b, 0, s, a);
    } else {
      if (edge) hipLaunchKernelGGL((stream_select_kernel<DT, 16, false, true>), g, b, 0, s, a);
      else hipLaunchKernelGGL((stream_select_kernel<DT, 16, false, false>), g, b, 0, s, a);
    }
  } else if (p.nt == kNTS) {
    // rows that start 16-byte aligned and fill their last vector have no
    // slots outside the row: the kernel without the edge handling
    const bool edge = ((uintptr_t)a.x % 16) != 0 || (a.cols * ElemT<DT>::ES) % 16 != 0;
    const dim3 g((unsigned)a.rows), b(kNTS);
    if (p.maxv == 19) {
      if (edge) hipLaunchKernelGGL((stream_select_kernel<DT, 19, SAMPLE, true>), g, b, 0, s, a);
      else hipLaunchKernelGGL((stream_select_kernel<DT, 19, SAMPLE, false>), g, b, 0, s, a);
    } else if (p.maxv == 16) {
      if (edge) hipLaunchKernelGGL((stream_select_kernel<DT, 16, SAMPLE, true>), g, b, 0, s, a);
      else hipLaunchKernelGGL((stream_select_kernel<DT, 16, SAMPLE, false>), g, b, 0, s, a);
    } else if (p.maxv == 8) {
      if (edge) hipLaunchKernelGGL((stream_select_kernel<DT, 8, SAMPLE, true>), g, b, 0, s, a);
      else hipLaunchKernelGGL((stream_select_kernel<DT, 8, SAMPLE, false>), g, b, 0, s, a);
    } else {
      if (edge) hipLaunchKernelGGL((stream_select_kernel<DT, 4, SAMPLE, true>), g, b, 0, s, a);
      else hipLaunchKernelGGL((stream_select_kernel<DT, 4, SAMPLE, false>), g, b, 0, s, a);
    }
    return launch_status(what);
  } else {
    if (p.maxv == 19) launch_a<DT, 19, kNT, SAMPLE>(a, s);
    else if (p.maxv == 16) launch_a<DT, 16, kNT, SAMPLE>(a, s);
    else if (p.maxv == 8) launch_a<DT, 8, kNT, SAMPLE>(a, s);
    else launch_a<DT, 4, kNT, SAMPLE>(a, s);
  }
  int st = launch_status(what);
  if (st || a0.nseg == 1) return st;
  if (!SAMPLE && !a0.lists_only && a0.k <= kWave && a0.nseg <= 2)
    hipLaunchKernelGGL((seg_merge64_pair_kernel<DT>), dim3((unsigned)a0.rows), dim3(kWave), 0, s, a0);
  else if (!SAMPLE && !a0.lists_only && a0.k <= kWave)
    hipLaunchKernelGGL((seg_merge64_kernel<DT>), dim3((unsigned)a0.rows), dim3(kMergeNT), 0, s, a0);
  else
    hipLaunchKernelGGL((seg_merge_kernel<DT, SAMPLE>), dim3((unsigned)a0.rows), dim3(kMergeNT), 0, s, a0);
  return launch_status(what);
}

// Sorted top-128 composites (select key << 32 | ~column) of every segment of
// every row into lists[rows][nseg][128], for callers that build on
// per-segment candidates (the binned top-k).  Segments are 256 threads x maxv
// vectors, maxv in {4, 8, 16}; a row is cut into at least min_seg segments
// when its length allows, at most kMaxSeg.  Returns kUnsupported when the row
// needs more segments than that.
int segment_lists_plan(int64_t rows, int64_t cols, int dt, int min_seg, int* nseg_out, int* maxv_out,
                       int64_t* vps_out) {
  const int vec = dt == kF32 ? 4 : 8;
  const int64_t nv = (cols + 2 * (vec - 1)) / vec;  // covers any row misalignment
  // 19 vectors per thread when that puts every segment in one residency
  // round (rows * nseg <= kTargetBlocks) where 16 would not, as plan_rows does
  {
    const int64_t n16 = (nv + (int64_t)kNT * 16 - 1) / ((int64_t)kNT * 16);
    const int64_t per19 = (int64_t)kNT * 19;
    const int64_t n19 = (nv + per19 - 1) / per19;
    if (rows * n16 > kTargetBlocks && rows * n19 <= kTargetBlocks && n19 >= min_seg && n19 >= 2 &&
        n19 <= kMaxSeg) {
      *nseg_out = (int)n19;
      *maxv_out = 19;
      *vps_out = per19;
      return kOk;
    }
  }
  int64_t nseg = (nv + (int64_t)kNT * 16 - 1) / ((int64_t)kNT * 16);
  if (nseg < min_seg) nseg = min_seg;
  if (nseg > nv) nseg = nv;
  if (nseg < 1) nseg = 1;
  if (nseg > kMaxSeg) return kUnsupported;
  const int64_t vps = (nv + nseg - 1) / nseg;
  int maxv = 4;
  while ((int64_t)kNT * maxv < vps) maxv *= 2;
  if (maxv > 16) return kUnsupported;
  *nseg_out = (int)((nv + vps - 1) / vps);
  *maxv_out = maxv;
  *vps_out = vps;
  return kOk;
}

int launch_segment_lists(const void* x, int dt, int64_t rows, int64_t cols, int nseg, int maxv, int64_t vps,
                         uint64_t* lists, hipStream_t s) {
  SelArgs a = {};
  a.x = x;
  a.rows = rows;
  a.cols = cols;
  a.k = kRun;
  a.nseg = nseg;
  a.vps = vps;
  a.ws_lists = lists;
  a.lists_only = 1;
  if (dt == kF32) {
    if (maxv == 19) launch_a<kF32, 19, kNT, false>(a, s);
    else if (maxv == 16) launch_a<kF32, 16, kNT, false>(a, s);
    else if (maxv == 8) launch_a<kF32, 8, kNT, false>(a, s);
    else launch_a<kF32, 4, kNT, false>(a, s);
  } else {
    if (maxv == 19) launch_a<kBF16, 19, kNT, false>(a, s);
    else if (maxv == 16) launch_a<kBF16, 16, kNT, false>(a, s);
    else if (maxv == 8) launch_a<kBF16, 8, kNT, false>(a, s);
    else launch_a<kBF16, 4, kNT, false>(a, s);
  }
  return launch_status("segment lists");
}

// ---------------------------------------------------------------------------
// Short rows (at most 2048 elements): every row sorted whole.  A 1024-thread
// select workgroup per row spends its fixed latency on a few hundred
// elements (f32, k = 8: [65536, 128] 1444 us, [65536, 512] 1703 us,
// [32768, 1024] 1051 us that way).  Records order the output ascending:
// (~select key) << 32 | column, the select key ordering values as the
// reference's strict `>` admits them (top_k.py:64: -0 == +0, NaN below -inf),
// ties by lowest column; padding records (all ones) go last.  Values at or
// below finfo(dtype).min, and NaNs, come out as finfo.min.
//   * rows of at most 32: one thread per row, a register bitonic network;
//   * longer rows: block_bitonic_sort_c over P = 64 .. 2048 slots, E records
//     per thread (one wave up to P = 512, then 128 and 256 threads).
// ---------------------------------------------------------------------------
constexpr int kTopkShortCols = 2048;

// Whole-row sorts pay off at any row count up to 256 elements; beyond that
// only with many rows, where the select kernel's per-row latency adds up
// (f32, k = 8, select -> sort: [65536, 512] 1711 -> 182 us, [32768, 1024]
// 1056 -> 223, [16384, 2048] 332 -> 271, [4096, 2048] 81 -> 80; few rows
// lose: [64, 1024] 10.3 -> 12.0, [256, 2048] 6.7 -> 14.8, [1024, 2048]
// k = 64 20.9 -> 28.9).
static bool topk_short_route(int64_t rows, int64_t cols) {
  return cols <= 256 || (cols <= 1024 && rows >= 512) || (cols <= kTopkShortCols && rows >= 8192);
}

__device__ __forceinline__ uint32_t topk_select_key(uint32_t b) {  // b: float32 bits
  const uint32_t a = b & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return 1u;
  if (a == 0u) return 0x80000000u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

template <int DT>
__device__ __forceinline__ uint32_t topk_f32_bits(const void* x, int64_t i) {
  return DT == kBF16 ? (uint32_t)((const uint16_t*)x)[i] << 16 : ((const uint32_t*)x)[i];
}

// Output position i of a row: positions >= k_rows[row] (when k_rows is
// given) keep the index and take the replacement value (float32 bits).
struct TopkShortOut {
  void* vals;
  int32_t* idx;
  const int32_t* k_rows;
  uint32_t replace_bits;
};

template <int DT>
__device__ __forceinline__ void topk_short_out(uint64_t rec, const void* x, int64_t base, int64_t row, int i, int k,
                                               const TopkShortOut& ot) {
  const int64_t o = row * k + i;
  void* out_vals = ot.vals;
  int32_t* out_idx = ot.idx;
  const uint32_t col = (uint32_t)rec;
  uint32_t b = topk_f32_bits<DT>(x, base + col);
  const uint32_t kmin = topk_select_key(DT == kBF16 ? 0xFF7F0000u : 0xFF7FFFFFu);
  if (topk_select_key(b) <= kmin) b = DT == kBF16 ? 0xFF7F0000u : 0xFF7FFFFFu;
  if (ot.k_rows && i >= ot.k_rows[row]) b = ot.replace_bits;
  out_idx[o] = (int32_t)col;
  if (DT == kBF16) ((uint16_t*)out_vals)[o] = (uint16_t)(b >> 16);
  else ((uint32_t*)out_vals)[o] = b;
}

template <int DT, int NC>
__global__ __launch_bounds__(256) void topk_short_thread_kernel(const void* __restrict__ x, int64_t rows, int cols,
                                                                int k, TopkShortOut ot) {
  const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  const int64_t base = row * cols;
  uint64_t v[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i)
    v[i] = i < cols ? ((uint64_t)~topk_select_key(topk_f32_bits<DT>(x, base + i)) << 32) | (uint32_t)i : ~0ull;
#pragma unroll
  for (int kk = 2; kk <= NC; kk <<= 1) {
#pragma unroll
    for (int j = kk >> 1; j > 0; j >>= 1) {
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const int o = i ^ j;
        if (o > i) {
          const uint64_t a = v[i], b = v[o];
          const bool sw = (i & kk) == 0 ? a > b : a < b;
          v[i] = sw ? b : a;
          v[o] = sw ? a : b;
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NC; ++i)
    if (i < k) topk_short_out<DT>(v[i], x, base, row, i, k, ot);
}

template <int DT, int P, int E>
__global__ __launch_bounds__(P / E) void topk_short_block_kernel(const void* __restrict__ x, int cols, int k,
                                                                 TopkShortOut ot) {
  __shared__ uint64_t lds[P];
  const int64_t row = blockIdx.x;
  const int64_t base = row * cols;
  const int t = threadIdx.x;
  uint64_t v[E];
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int i = t * E + r;
    v[r] = i < cols ? ((uint64_t)~topk_select_key(topk_f32_bits<DT>(x, base + i)) << 32) | (uint32_t)i : ~0ull;
  }
  block_bitonic_sort_c<uint64_t, E, P, false>(v, lds);
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int i = t * E + r;
    if (i < k) topk_short_out<DT>(v[r], x, base, row, i, k, ot);
  }
}

template <int DT>
static int launch_topk_short(const void* x, int64_t rows, int64_t cols, int k, const TopkShortOut& ot,
                             hipStream_t s) {
  const int c = (int)cols;
  if (cols <= 32) {
    const unsigned grid = (unsigned)((rows + 255) / 256);
    if (cols <= 16)
      hipLaunchKernelGGL((topk_short_thread_kernel<DT, 16>), dim3(grid), dim3(256), 0, s, x, rows, c, k, ot);
    else
      hipLaunchKernelGGL((topk_short_thread_kernel<DT, 32>), dim3(grid), dim3(256), 0, s, x, rows, c, k, ot);
  } else if (cols <= 64) {
    hipLaunchKernelGGL((topk_short_block_kernel<DT, 64, 1>), dim3((unsigned)rows), dim3(64), 0, s, x, c, k, ot);
  } else if (cols <= 128) {
    hipLaunchKernelGGL((topk_short_block_kernel<DT, 128, 2>), dim3((unsigned)rows), dim3(64), 0, s, x, c, k, ot);
  } else if (cols <= 256) {
    hipLaunchKernelGGL((topk_short_block_kernel<DT, 256, 4>), dim3((unsigned)rows), dim3(64), 0, s, x, c, k, ot);
  } else if (cols <= 512) {
    hipLaunchKernelGGL((topk_short_block_kernel<DT, 512, 8>), dim3((unsigned)rows), dim3(64), 0, s, x, c, k, ot);
  } else if (cols <= 1024) {
    hipLaunchKernelGGL((topk_short_block_kernel<DT, 1024, 8>), dim3((unsigned)rows), dim3(128), 0, s, x, c, k, ot);
  } else {
    hipLaunchKernelGGL((topk_short_block_kernel<DT, 2048, 8>), dim3((unsigned)rows), dim3(256), 0, s, x, c, k, ot);
  }
  return launch_status("top-k (short rows)");
}

static int check_common(const void* x, int dt, int64_t rows, int64_t cols) {
  if (!x) { set_error("null input pointer"); return kInvalidArgument; }
  if (dt != kF32 && dt != kBF16) { set_error("dtype %d not supported (f32=0, bf16=1)", dt); return kUnsupported; }
  if (rows < 0 || cols <= 0) { set_error("bad shape [%lld, %lld]", (long long)rows, (long long)cols); return kInvalidArgument; }
  // workgroups per launch: rows x segments (at most 64) stay within the grid's 2^31 - 1
  if (rows > ((int64_t)1 << 31) / 64 - 1) { set_error("rows %lld exceed the grid limit", (long long)rows); return kUnsupported; }
  if (cols >= (int64_t)1 << 31) { set_error("cols must fit int32 indices"); return kInvalidArgument; }
  return kOk;
}

// ---------------------------------------------------------------------------
// int32 logits (the reference's top-k is dtype-generic: bins start at
// iinfo.min and admit only strictly greater values, utils.py:48-56,
// top_k.py:64,241-243).  The exact answer under the lowest-index tie rule is
// the first k of the row's stable descending sort: values descending, equal
// values by ascending index, and iinfo.min elements (never admitted, so they
// fill the tail with the dtype's min) last in index order.  The int32 row sort
// (sort_rows.hip) writes that permutation into the workspace; this kernel
// gathers the first k columns.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void topk_from_perm_kernel(const int32_t* __restrict__ x,
                                                             const int32_t* __restrict__ perm, int64_t cols, int k,
                                                             int32_t* __restrict__ out_vals,
                                                             int32_t* __restrict__ out_idx,
                                                             const int32_t* __restrict__ k_rows, int has_replace,
                                                             int32_t replace_val, int64_t n) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t r = e / k;
    const int j = (int)(e - r * k);
    const int32_t p = perm[r * cols + j];  // in [0, cols): a permutation of the row
    out_idx[e] = p;
    out_vals[e] = (has_replace && j >= k_rows[r]) ? replace_val : x[r * cols + p];
  }
}

static size_t topk_i32_ws(int64_t rows, int64_t cols) {
  return align_up((size_t)rows * (size_t)cols * 4, 256) + sort_wide_workspace_bytes(rows, cols);
}

static int topk_i32(const void* x, int64_t rows, int64_t cols, int64_t k, const int32_t* k_rows, double replace_val,
                    void* out_vals, int32_t* out_idx, void* workspace, size_t workspace_bytes, hipStream_t stream,
                    const char* what) {
  const size_t need = topk_i32_ws(rows, cols);
  if (!workspace || workspace_bytes < need) {
    set_error("workspace of %zu bytes is smaller than the %zu required", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  int32_t* perm = (int32_t*)workspace;
  const size_t perm_bytes = align_up((size_t)rows * (size_t)cols * 4, 256);
  int st = tallax_sort_rows_ws(x, kI32, rows, cols, /*descending=*/1, /*ties_descending=*/0, nullptr, perm, nullptr,
                               0, nullptr, 0, nullptr, 0, (char*)workspace + perm_bytes, workspace_bytes - perm_bytes,
                               stream);
  if (st) return st;
  // int32 outputs take replace_val converted toward zero, saturated at the int32 range (NaN -> 0)
  double rv = replace_val != replace_val ? 0.0 : replace_val;
  rv = rv < -2147483648.0 ? -2147483648.0 : (rv > 2147483647.0 ? 2147483647.0 : rv);
  const int64_t n = rows * k;
  const int64_t blocks = (n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536;
  hipLaunchKernelGGL(topk_from_perm_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, (const int32_t*)x, perm,
                     cols, (int)k, (int32_t*)out_vals, out_idx, k_rows, k_rows ? 1 : 0, (int32_t)rv, n);
  return launch_status(what);
}

}  // namespace tx

using namespace tx;

extern "C" {

size_t tallax_topk_workspace_size(int64_t rows, int64_t cols, int64_t k, int dtype) {
  Plan p;
  if (k < 1 || k > kMaxK || rows < 0 || cols <= 0) return 0;
  if (dtype == kI32) return topk_i32_ws(rows, cols);
  if (dtype != kF32 && dtype != kBF16) return 0;
  if (plan_rows(rows, cols, dtype, &p) != kOk) return 0;
  return ws_bytes_for(rows, p);
}

int tallax_topk(const void* x, int dtype, int64_t rows, int64_t cols, int64_t k, void* out_vals,
                int32_t* out_idx, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  int st = check_common(x, dtype == kI32 ? kF32 : dtype, rows, cols);
  if (st) return st;
  if (k < 1 || k > kMaxK) { set_error("k=%lld outside [1, %d]", (long long)k, kMaxK); return k > kMaxK ? kUnsupported : kInvalidArgument; }
  if (k > cols) { set_error("k=%lld exceeds row length %lld", (long long)k, (long long)cols); return kInvalidArgument; }
  if (!out_vals || !out_idx) { set_error("null output pointer"); return kInvalidArgument; }
  if (rows == 0) return kOk;
  if (dtype == kI32)
    return topk_i32(x, rows, cols, k, nullptr, 0.0, out_vals, out_idx, workspace, workspace_bytes, stream, "tallax_topk");
  if (topk_short_route(rows, cols)) {
    const TopkShortOut ot = {out_vals, out_idx, nullptr, 0u};
    return dtype == kF32 ? launch_topk_short<kF32>(x, rows, cols, (int)k, ot, stream)
                         : launch_topk_short<kBF16>(x, rows, cols, (int)k, ot, stream);
  }
  Plan p;
  st = plan_rows(rows, cols, dtype, &p);
  if (st) return st;
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
  return dtype == kF32 ? launch_select<kF32, false>(a, p, stream, "tallax_topk")
                       : launch_select<kBF16, false>(a, p, stream, "tallax_topk");
}

int tallax_topk_replace(const void* x, int dtype, int64_t rows, int64_t cols, int64_t k, const int32_t* k_rows,
                        double replace_val, void* out_vals, int32_t* out_idx, void* workspace,
                        size_t workspace_bytes, hipStream_t stream) {
  int st = check_common(x, dtype == kI32 ? kF32 : dtype, rows, cols);
  if (st) return st;
  if (k < 1 || k > kMaxK) { set_error("k=%lld outside [1, %d]", (long long)k, kMaxK); return k > kMaxK ? kUnsupported : kInvalidArgument; }
  if (k > cols) { set_error("k=%lld exceeds row length %lld", (long long)k, (long long)cols); return kInvalidArgument; }
  if (!out_vals || !out_idx || !k_rows) { set_error("null pointer argument"); return kInvalidArgument; }
  if (rows == 0) return kOk;
  if (dtype == kI32)
    return topk_i32(x, rows, cols, k, k_rows, replace_val, out_vals, out_idx, workspace, workspace_bytes, stream,
                    "tallax_topk_replace");
  if (topk_short_route(rows, cols)) {
    const float rf = (float)replace_val;
    uint32_t rb;
    const float rd = dtype == kBF16 ? round_to_bf16(rf) : rf;
    memcpy(&rb, &rd, sizeof(rb));
    const TopkShortOut ot = {out_vals, out_idx, k_rows, rb};
    return dtype == kF32 ? launch_topk_short<kF32>(x, rows, cols, (int)k, ot, stream)
                         : launch_topk_short<kBF16>(x, rows, cols, (int)k, ot, stream);
  }
  Plan p;
  st = plan_rows(rows, cols, dtype, &p);
  if (st) return st;
  const size_t need = ws_bytes_for(rows, p);
  if (workspace_bytes < need || (need && !workspace)) {
    set_error("workspace of %zu bytes is smaller than the %zu required", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  SelArgs a = {};
  a.x = x; a.rows = rows; a.cols = cols; a.k = (int)k;
  a.nseg = p.nseg; a.vps = p.vps;
  a.out_vals = out_vals; a.out_idx = out_idx;
  a.k_rows = k_rows;
  const float rf = (float)replace_val;
  a.replace_in_dtype = dtype == kBF16 ? round_to_bf16(rf) : rf;
  a.ws_lists = (uint64_t*)workspace;
  return dtype == kF32 ? launch_select<kF32, false>(a, p, stream, "tallax_topk_replace")
                       : launch_select<kBF16, false>(a, p, stream, "tallax_topk_replace");
}

size_t tallax_sample_workspace_size(int64_t rows, int64_t vocab, int dtype) {
  return tallax_topk_workspace_size(rows, vocab, kMaxK, dtype);
}

}  // extern "C"

// The fused sampler with its workspace given (workspace != nullptr or none
// needed) or, for the no-allocation entry point (use_scratch), the device
// scratch array below.
static int fused_sample(const void* logits, int dtype, int64_t rows, int64_t vocab, const int32_t* top_k,
                        const float* top_p, const float* temperature, const uint32_t* rng_key, int64_t dim0_offset,
                        double replace_val, int32_t* out_tokens, void* workspace, size_t workspace_bytes,
                        hipStream_t stream, bool use_scratch);

// Scratch of tallax_fused_topk_topp_sample_noalloc: the per-segment candidate
// lists of segmented rows (rows x segments x 1 KiB).  Every GPU the library
// runs on holds its own copy until the process ends.  In host code the array's
// name is not a device address: kernels get the per-device address from
// hipGetSymbolAddress (scratch_address).  Calls on one GPU share it, so calls
// that overlap there race; no call reads bytes it did not write itself, so
// nothing needs clearing between calls.
constexpr size_t kSampleScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kSampleScratchBytes];

constexpr int kMaxDevices = 64;

// Device address of `scratch` on the device of `stream` (the current device
// for the null stream), looked up once per device with that device current.
// The lookup (hipSetDevice, hipGetSymbolAddress) is not made while `stream`
// is capturing: a device's first call under capture returns
// TALLAX_UNSUPPORTED and leaves the capture untouched, so a capturing caller
// makes one call per device before it captures.  Later calls only read the
// cached address and are capturable.
static int scratch_address(hipStream_t stream, void** out) {
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess) {
    set_error("hipGetDevice failed");
    return kHipError;
  }
  int dev = cur;
  if (stream && hipStreamGetDevice(stream, &dev) != hipSuccess) {
    set_error("hipStreamGetDevice failed");
    return kHipError;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("device %d outside the %d this build tracks", dev, kMaxDevices);
    return kUnsupported;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
      set_error("hipStreamIsCapturing failed");
      return kHipError;
    }
    if (cs != hipStreamCaptureStatusNone) {
      set_error("the first no-allocation call on device %d is under stream capture; make one call on that device "
                "before capturing (it looks up the device address of the scratch array)", dev);
      return kUnsupported;
    }
    if (dev != cur && hipSetDevice(dev) != hipSuccess) {
      set_error("hipSetDevice(%d) failed", dev);
      return kHipError;
    }
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p) {
      set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
      return kHipError;
    }
    addr[dev] = p;
  }
  *out = addr[dev];
  return kOk;
}

extern "C" {

int tallax_fused_topk_topp_sample(const void* logits, int dtype, int64_t rows, int64_t vocab,
                                  const int32_t* top_k, const float* top_p, const float* temperature,
                                  const uint32_t* rng_key, int64_t dim0_offset, double replace_val,
                                  int32_t* out_tokens, void* workspace, size_t workspace_bytes,
                                  hipStream_t stream) {
  return fused_sample(logits, dtype, rows, vocab, top_k, top_p, temperature, rng_key, dim0_offset, replace_val,
                      out_tokens, workspace, workspace_bytes, stream, false);
}

int tallax_fused_topk_topp_sample_noalloc(const void* logits, int dtype, int64_t rows, int64_t vocab,
                                          const int32_t* top_k, const float* top_p, const float* temperature,
                                          const uint32_t* rng_key, int64_t dim0_offset, double replace_val,
                                          int32_t* out_tokens, hipStream_t stream) {
  return fused_sample(logits, dtype, rows, vocab, top_k, top_p, temperature, rng_key, dim0_offset, replace_val,
                      out_tokens, nullptr, 0, stream, true);
}

}  // extern "C"

static int fused_sample(const void* logits, int dtype, int64_t rows, int64_t vocab, const int32_t* top_k,
                        const float* top_p, const float* temperature, const uint32_t* rng_key, int64_t dim0_offset,
                        double replace_val, int32_t* out_tokens, void* workspace, size_t workspace_bytes,
                        hipStream_t stream, bool use_scratch) {
  int st = check_common(logits, dtype, rows, vocab);
  if (st) return st;
  if (vocab < kMaxK) { set_error("vocab %lld < 128 is not supported by the fused sampler", (long long)vocab); return kUnsupported; }
  if (!top_k || !top_p || !temperature || !rng_key || !out_tokens) { set_error("null pointer argument"); return kInvalidArgument; }
  if (rows == 0) return kOk;
  Plan p;
  st = plan_rows(rows, vocab, dtype, &p);
  if (st) return st;
  const size_t need = ws_bytes_for(rows, p);
  if (use_scratch) {
    if (need > kSampleScratchBytes) {
      set_error("[%lld, %lld] needs %zu bytes of scratch; the no-allocation sampler holds %zu (pass a workspace to "
                "tallax_fused_topk_topp_sample instead)", (long long)rows, (long long)vocab, need,
                kSampleScratchBytes);
      return kUnsupported;
    }
    if (need) {
      st = scratch_address(stream, &workspace);
      if (st) return st;
      workspace_bytes = kSampleScratchBytes;
    }
  } else if (workspace_bytes < need || (need && !workspace)) {
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
  return dtype == kF32 ? launch_select<kF32, true>(a, p, stream, "tallax_fused_topk_topp_sample")
                       : launch_select<kBF16, true>(a, p, stream, "tallax_fused_topk_topp_sample");
}

extern "C" {

size_t tallax_shard_candidates_workspace_size(int64_t rows, int64_t cols, int dtype) {
  return tallax_topk_workspace_size(rows, cols, kMaxK, dtype);
}

int tallax_shard_candidates(const void* x, int dtype, int64_t rows, int64_t cols, int64_t col_offset,
                            uint64_t* candidates, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  int st = check_common(x, dtype, rows, cols);
  if (st) return st;
  if (cols < kMaxK) { set_error("a shard of %lld < 128 columns is not supported", (long long)cols); return kUnsupported; }
  if (col_offset < 0 || col_offset + cols >= (int64_t)1 << 31) { set_error("column offset %lld out of range", (long long)col_offset); return kInvalidArgument; }
  if (!candidates) { set_error("null pointer argument"); return kInvalidArgument; }
  if (rows == 0) return kOk;
  Plan p;
  st = plan_rows(rows, cols, dtype, &p);
  if (st) return st;
  const size_t need = ws_bytes_for(rows, p);
  if (workspace_bytes < need || (need && !workspace)) {
    set_error("workspace of %zu bytes is smaller than the %zu required", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  SelArgs a = {};
  a.x = x; a.rows = rows; a.cols = cols; a.k = kMaxK;
  a.nseg = p.nseg; a.vps = p.vps;
  a.lists_only = 1;
  a.col_offset = col_offset;
  // one segment: the segment kernel writes the row's list itself; more: per-segment
  // lists in the workspace, merged into the output by the merge kernel
  a.ws_lists = p.nseg == 1 ? candidates : (uint64_t*)workspace;
  a.out_lists = candidates;
  return dtype == kF32 ? launch_select<kF32, false>(a, p, stream, "tallax_shard_candidates")
                       : launch_select<kBF16, false>(a, p, stream, "tallax_shard_candidates");
}

int tallax_sample_from_candidates(const uint64_t* candidates, int64_t nlists, int dtype, int64_t rows,
                                  int64_t vocab, const int32_t* top_k, const float* top_p, const float* temperature,
                                  const uint32_t* rng_key, int64_t dim0_offset, double replace_val,
                                  int32_t* out_tokens, hipStream_t stream) {
  if (!candidates || !top_k || !top_p || !temperature || !rng_key || !out_tokens) { set_error("null pointer argument"); return kInvalidArgument; }
  if (dtype != kF32 && dtype != kBF16) { set_error("dtype %d not supported (f32=0, bf16=1)", dtype); return kUnsupported; }
  if (nlists < 1 || nlists > kMaxSeg) { set_error("%lld candidate lists per row: 1 to %d are supported", (long long)nlists, kMaxSeg); return nlists < 1 ? kInvalidArgument : kUnsupported; }
  if (rows < 0 || vocab < kMaxK || vocab >= (int64_t)1 << 31) { set_error("bad shape: rows %lld, vocab %lld", (long long)rows, (long long)vocab); return kInvalidArgument; }
  if (rows > 2147483647) { set_error("too many rows"); return kUnsupported; }
  if (rows == 0) return kOk;
  SelArgs a = {};
  a.rows = rows; a.cols = vocab; a.k = kMaxK;
  a.nseg = (int)nlists;
  a.ws_lists = const_cast<uint64_t*>(candidates);
  a.top_k = top_k; a.top_p = top_p; a.temperature = temperature; a.rng_key = rng_key;
  a.dim0_offset = dim0_offset;
  const float rf = (float)replace_val;
  a.replace_f32 = rf;
  a.replace_in_dtype = dtype == kBF16 ? round_to_bf16(rf) : rf;
  a.out_tokens = out_tokens;
  if (dtype == kF32)
    hipLaunchKernelGGL((seg_merge_kernel<kF32, true>), dim3((unsigned)rows), dim3(kMergeNT), 0, stream, a);
  else
    hipLaunchKernelGGL((seg_merge_kernel<kBF16, true>), dim3((unsigned)rows), dim3(kMergeNT), 0, stream, a);
  return launch_status("tallax_sample_from_candidates");
}

int tallax_testing_select_plan(int64_t rows, int64_t cols, int dtype, int32_t* out) {
  if (!out || (dtype != kF32 && dtype != kBF16) || rows < 0 || cols <= 0) {
    set_error("bad arguments");
    return kInvalidArgument;
  }
  Plan p;
  const int st = plan_rows(rows, cols, dtype, &p);
  if (st) return st;
  out[0] = p.nt;
  out[1] = p.maxv;
  out[2] = p.nseg;
  out[3] = (int32_t)p.vps;
  return kOk;
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

int tallax_top_p_mask(const float* topk_logits, int64_t k, int64_t cols, const float* top_p, double replace_val,
                      float* out, hipStream_t stream) {
  if (!topk_logits || !top_p || !out) { set_error("null pointer argument"); return kInvalidArgument; }
  if (k < 1 || cols < 0) { set_error("bad extents k=%lld cols=%lld", (long long)k, (long long)cols); return kInvalidArgument; }
  if (k > kMaxK) { set_error("k=%lld > 128 candidates per column is not supported", (long long)k); return kUnsupported; }
  if (cols > 2147483647) { set_error("too many columns"); return kUnsupported; }
  if (cols == 0) return kOk;
  hipLaunchKernelGGL(top_p_mask_kernel, dim3((unsigned)cols), dim3(kWave), 0, stream, topk_logits, cols, (int)k,
                     top_p, (float)replace_val, out);
  return launch_status("tallax_top_p_mask");
}

}  // extern "C"
