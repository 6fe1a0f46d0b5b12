/*
 * tallax_hip.h -- C ABI of the MI355X (gfx950) sort / select / sample library.
 *
 * Conventions (every entry point):
 *   - All array arguments are DEVICE pointers to dense row-major buffers owned
 *     by the caller; scalars are passed by value.
 *   - Work is enqueued on `stream` only; nothing synchronizes the host and
 *     nothing allocates device memory.  Entry points that need scratch take a
 *     caller-provided `workspace` of at least `*_workspace_size(...)` bytes
 *     (0 when the work split needs none; no initial contents are required:
 *     every byte read is written earlier in the same call).  Calls that may
 *     run concurrently need distinct workspaces.
 *   - Return value: 0 on success, otherwise a TALLAX_* status code; the
 *     message of the last failure on the calling thread is returned by
 *     tallax_last_error().
 *   - dtype codes: TALLAX_F32 = 0, TALLAX_BF16 = 1, TALLAX_I32 = 2.
 *
 * Each entry point replaces one jit-wrapped Pallas call of the reference
 * (oliverdutton/tallax); the reference interface is cited above each
 * declaration as file:line.
 */
#ifndef TALLAX_HIP_H_
#define TALLAX_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* tallax_stream_t; /* == hipStream_t */

enum {
  TALLAX_OK = 0,
  TALLAX_INVALID_ARGUMENT = 1,
  TALLAX_UNSUPPORTED = 2,
  TALLAX_HIP_ERROR = 3,
  TALLAX_WORKSPACE_TOO_SMALL = 4,
};

enum { TALLAX_F32 = 0, TALLAX_BF16 = 1, TALLAX_I32 = 2 };

/* Message describing the last failure on this thread ("" if none). */
const char* tallax_last_error(void);

/* ABI revision of this header. */
int tallax_abi_version(void);

/* ------------------------------------------------------------------------
 * Exact top-k along the last axis.
 * Replaces tax.top_k(logits, k)  -- tallax/_src/top_k.py:516-567
 * (= top_dynamic_k(max_k=k, guarantee_convergence=True), top_k.py:372-514,
 * kernel dynamic_top_k_refs top_k.py:203-370).
 * x: [rows, cols] f32, bf16 or int32.  Outputs: out_vals [rows, k] (same
 * dtype, descending), out_idx [rows, k] int32; ties broken to the lowest
 * index.  1 <= k <= 128 (the reference raises NotImplementedError above 128,
 * top_k.py:438-439), k <= cols.  NaN, -inf and finfo(dtype).min are never
 * preferred over other values; slots that can only be filled by them hold
 * finfo(dtype).min, as the reference's bins do (top_k.py:241-243).  int32
 * rows (the reference's dtype-generic path, utils.py:48-56) are the first k
 * of the row's stable descending sort, iinfo.min entries last; their
 * workspace holds that sort's permutation (rows * cols * 4 bytes plus the
 * row sort's own workspace).
 * ---------------------------------------------------------------------- */
size_t tallax_topk_workspace_size(int64_t rows, int64_t cols, int64_t k, int dtype);
int tallax_topk(const void* x, int dtype, int64_t rows, int64_t cols, int64_t k, void* out_vals,
                int32_t* out_idx, void* workspace, size_t workspace_bytes, tallax_stream_t stream);

/* ------------------------------------------------------------------------
 * Exact top-k with per-row k and a replacement value: top_k(x, k) whose
 * positions >= k_rows[row] hold replace_val (in x's dtype).
 * The exact counterpart of top_dynamic_k(logits, k, max_k, replace_val)
 * -- tallax/_src/top_k.py:385-514 (replacement :365-369) -- for a run that
 * converges, under the lowest-index tie rule of tax.top_k.  Workspace as tallax_topk
 * (tallax_topk_workspace_size).  For int32 x, replace_val is converted toward
 * zero and saturated at the int32 range.
 * ---------------------------------------------------------------------- */
int tallax_topk_replace(const void* x, int dtype, int64_t rows, int64_t cols, int64_t k, const int32_t* k_rows,
                        double replace_val, void* out_vals, int32_t* out_idx, void* workspace,
                        size_t workspace_bytes, tallax_stream_t stream);

/* ------------------------------------------------------------------------
 * Binned top-k: top_dynamic_k.
 * Replaces top_dynamic_k -- tallax/_src/top_k.py:385-514 (kernel
 * dynamic_top_k_refs :203-370, binned_top_k :13-106, and with
 * guarantee_convergence the bin-packing merge of unconverged blocks,
 * _merge_unconverged_bins_top_k :108-200, invoked at :317-331).
 * x [rows, cols] f32/bf16/int32; k_rows [rows] int32 (per-row k <= max_k <= 128);
 * rows % block_token == 0; num_bins divides 1024; schedule: the strictly
 * increasing depths m (the reference's bins_topm_schedule without its
 * leading 0; the caller computes the automatic one), deepest <= 16 after
 * power-of-two bucketing.  guarantee_convergence != 0 with a last depth m
 * other than max_k needs m >= 2 and num_bins % 128 == 0 (the merge packs
 * the 2^ceil(log2(ceil(max_k / (m - 1)))) busiest bins).  Outputs:
 * out_vals [rows, max_k] (x's dtype), out_idx [rows, max_k] int32 (-1 where
 * fewer admissible elements exist; the merge can also return columns past
 * the row's end, with finfo.min, where the reference reads past it),
 * out_valid [1] int32 (0/1), out_depths [rows] int32, out_cutoff [rows] f32
 * (int32 for int32 x: the reference's cutoff is to_32bit_dtype(x.dtype),
 * top_k.py:465; the buffer is 4 bytes per row either way).  int32 x: bins
 * start at iinfo.min, the merge fills chosen bins with iinfo.min, and
 * replace_val is converted toward zero and saturated at the int32 range.
 * Workspace: tallax_top_dynamic_k_workspace_size bytes.
 * ---------------------------------------------------------------------- */
size_t tallax_top_dynamic_k_workspace_size(int64_t rows, int num_bins, const int32_t* schedule, int num_steps);
int tallax_top_dynamic_k(const void* x, int dtype, int64_t rows, int64_t cols, const int32_t* k_rows, int max_k,
                         int block_token, int num_bins, const int32_t* schedule, int num_steps,
                         int guarantee_convergence, int has_replace, double replace_val, void* out_vals,
                         int32_t* out_idx, int32_t* out_valid, int32_t* out_depths, float* out_cutoff,
                         void* workspace, size_t workspace_bytes, tallax_stream_t stream);

/* ------------------------------------------------------------------------
 * Fused vLLM-style sampler: top-k (per-row k, clamped to 128) -> top-p ->
 * temperature -> Gumbel-max, one token per row, in one kernel launch.
 * Replaces sampling.sample(rng_key, logits, tpu_sampling_metadata)
 *   -- tallax/_src/sampling.py:331-343, i.e. _top_k_with_sharding
 *   (sampling.py:271-328, single device: top_dynamic_k(max_k=128,
 *   num_bins=256, bins_topm_schedule=(5,9), guarantee_convergence=True,
 *   replace_val)) followed by top_p_and_sample (sampling.py:210-269).
 * logits [rows, vocab] f32/bf16; top_k [rows] int32; top_p, temperature
 * [rows] f32; rng_key: 2 uint32 words of threefry key data (device);
 * dim0_offset: global row offset of this shard for the noise counters
 * (sampling.py:249-251); replace_val: the value written over filtered
 * candidates (the reference passes -1e12).  out_tokens [rows] int32.
 * vocab >= 128.
 * ---------------------------------------------------------------------- */
size_t tallax_sample_workspace_size(int64_t rows, int64_t vocab, int dtype);
int tallax_fused_topk_topp_sample(const void* logits, int dtype, int64_t rows, int64_t vocab,
                                  const int32_t* top_k, const float* top_p, const float* temperature,
                                  const uint32_t* rng_key, int64_t dim0_offset, double replace_val,
                                  int32_t* out_tokens, void* workspace, size_t workspace_bytes,
                                  tallax_stream_t stream);

/* ------------------------------------------------------------------------
 * The fused sampler with no workspace argument and no allocation.
 * NO COUNTERPART IN THE REFERENCE: for callers that cannot allocate device
 * memory or pass a workspace (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments and results as
 * tallax_fused_topk_topp_sample; the candidate lists of rows split into
 * segments or whole-row parts go to a static device array of 16 MiB that
 * each GPU holds until the process ends (it calls no hipMalloc/hipFree).
 * Inputs whose lists need more (rows x lists x 1 KiB; e.g. f32 rows of 151936
 * columns beyond about 1600 rows) return TALLAX_UNSUPPORTED before any
 * launch.  All
 * calls on one GPU share the array: calls that overlap on one GPU race.
 * The first call on a device looks up the array's device address; made
 * while `stream` is capturing, that call returns TALLAX_UNSUPPORTED and
 * leaves the capture untouched, so a capturing caller makes one call per
 * device first.  Later calls capture and replay like the other entry points.
 * ---------------------------------------------------------------------- */
int tallax_fused_topk_topp_sample_noalloc(const void* logits, int dtype, int64_t rows, int64_t vocab,
                                          const int32_t* top_k, const float* top_p, const float* temperature,
                                          const uint32_t* rng_key, int64_t dim0_offset, double replace_val,
                                          int32_t* out_tokens, tallax_stream_t stream);

/* ------------------------------------------------------------------------
 * Wide-candidate sampler: sampling.sample (tallax/_src/sampling.py:331-343)
 * with the top-k width max_k lifted from the reference's 128
 * (sampling.py:283-290, top_k.py:438-439) to any max_k in [1, 1024], so that
 * per-row top_k up to 1024 is honoured instead of clamped.  Same algorithm
 * otherwise: exact top-max_k (value descending, ties to the lowest index),
 * positions >= top_k[row] replaced by replace_val in the logits dtype, then
 * top_p_and_sample (sampling.py:65-115) over the max_k candidates.  With
 * max_k = 128 the tokens equal tallax_fused_topk_topp_sample's.
 * out_tokens [rows] (or null); out_idx [rows, max_k] int32 and out_vals
 * [rows, max_k] f32 (each optional) receive the candidates before the k
 * mask.  max_k <= vocab.  No workspace.
 * ---------------------------------------------------------------------- */
int tallax_sample_wide(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t max_k,
                       const int32_t* top_k, const float* top_p, const float* temperature,
                       const uint32_t* rng_key, int64_t dim0_offset, double replace_val, int32_t* out_tokens,
                       int32_t* out_idx, float* out_vals, tallax_stream_t stream);

/* ------------------------------------------------------------------------
 * Vocabulary-sharded sampling, the two compute steps of the reference's
 * partitioned sampler (tallax/_src/sampling.py:300-321: per-shard
 * _top_k_arrays(logits, 128), indices to the global frame, all_gather, then
 * bitonic_top_k of the gathered lists, the k mask and top_p_and_sample).
 * tallax_shard_candidates: the shard x [rows, cols] (f32/bf16, cols >= 128,
 * its first column is global column col_offset) -> candidates [rows, 128]
 * u64, its sorted top-128 as composites (select key << 32 | ~global column;
 * larger = earlier, ties to the lowest column).  Workspace:
 * tallax_shard_candidates_workspace_size bytes (0 for whole-row plans).
 * tallax_sample_from_candidates: candidates [rows, nlists, 128] u64 (the
 * lists of nlists <= 32 shards side by side per row, i.e. what an all-gather
 * along axis 1 gives) -> out_tokens [rows] int32: their merged top-128 (the
 * global top-128, ties to the lowest column), positions >= top_k[row]
 * replaced by replace_val in the logits dtype, then the sampler tail with
 * vocab = the total vocabulary.  The tokens equal tallax_fused_topk_topp_sample
 * on the unsharded logits.
 * ---------------------------------------------------------------------- */
size_t tallax_shard_candidates_workspace_size(int64_t rows, int64_t cols, int dtype);
int tallax_shard_candidates(const void* x, int dtype, int64_t rows, int64_t cols, int64_t col_offset,
                            uint64_t* candidates, void* workspace, size_t workspace_bytes, tallax_stream_t stream);
int tallax_sample_from_candidates(const uint64_t* candidates, int64_t nlists, int dtype, int64_t rows,
                                  int64_t vocab, const int32_t* top_k, const float* top_p, const float* temperature,
                                  const uint32_t* rng_key, int64_t dim0_offset, double replace_val,
                                  int32_t* out_tokens, tallax_stream_t stream);

/* ------------------------------------------------------------------------
 * Top-p mask over already-selected, descending candidates, along axis 0.
 * Replaces top_p_mask(*, topk_logits, p, replace_val, axis=0) --
 * tallax/_src/sampling.py:25-62: probs = exp(l - l[0]) / sum, inclusive
 * cumsum in the (8, 128)-tile order of cumsum_arrays (cumsum.py:32-63),
 * t = #(cumsum < p), threshold l[t] (0.0 when t == k, the out-of-range
 * gather), keep l >= threshold, replace_val elsewhere.
 * topk_logits, out [k, cols] f32 (column b sorted descending); top_p [cols]
 * f32; 1 <= k <= 128 (the sampler's candidate count, sampling.py:283-290).
 * ---------------------------------------------------------------------- */
int tallax_top_p_mask(const float* topk_logits, int64_t k, int64_t cols, const float* top_p, double replace_val,
                      float* out, tallax_stream_t stream);

/* ------------------------------------------------------------------------
 * Top-p filter + temperature + Gumbel-max sampling over already-selected,
 * descending candidates.
 * Replaces top_p_and_sample(topk_logits, topk_idx, rng_key, top_p,
 * temperature, *, vocab_size, replace_val) -- tallax/_src/sampling.py:210-269
 * (kernel top_p_and_sample_refs/arrays, sampling.py:65-153).
 * topk_logits [rows, k] f32/bf16, topk_idx [rows, k] int32, k <= 128.
 * ---------------------------------------------------------------------- */
int tallax_top_p_and_sample(const void* topk_logits, int dtype, const int32_t* topk_idx, int64_t rows,
                            int64_t k, const uint32_t* rng_key, const float* top_p,
                            const float* temperature, int64_t vocab_size, double replace_val,
                            int64_t dim0_offset, int32_t* out_tokens, tallax_stream_t stream);

/* ------------------------------------------------------------------------
 * Gather along an axis: out = values[indices] along `axis` (0 or 1), 0 where
 * the index is negative or >= the values' extent (no negative wrap).
 * Replaces tumpy.take_along_axis(arr, indices, axis)
 *   -- tallax/tumpy.py:99-112, tallax/_src/gather.py:59-83
 *   (kernel take_along_axis_arrays, gather.py:11-45).
 * values [vrows, vcols] f32/bf16/int32; indices [irows, icols] int32;
 * out [irows, icols] in the values' dtype.  axis 1 needs vrows == irows,
 * axis 0 needs vcols == icols.
 * ---------------------------------------------------------------------- */
int tallax_take_along_axis(const void* values, int dtype, int64_t vrows, int64_t vcols, const int32_t* indices,
                           int64_t irows, int64_t icols, int axis, void* out, tallax_stream_t stream);

/* ------------------------------------------------------------------------
 * Inclusive cumulative sum along `axis` (0 or 1), optionally reversed, in the
 * reference's summation order: Hillis-Steele inside (8, 128) tiles, then the
 * running total of earlier tiles added sequentially.
 * Replaces tax.cumsum(arr, axis, reverse) -- tallax/_src/cumsum.py:75-101
 *   (kernel cumsum_arrays, cumsum.py:32-63).
 * x, out [rows, cols] f32 or int32 (int32 adds wrap); out must not overlap x
 * (tile totals are staged in out; overlap returns TALLAX_INVALID_ARGUMENT).
 * ---------------------------------------------------------------------- */
int tallax_cumsum(const void* x, int dtype, int64_t rows, int64_t cols, int axis, int reverse, void* out,
                  tallax_stream_t stream);

/* ------------------------------------------------------------------------
 * Row-wise sort by one key: the kernel under tax.sort / tumpy.sort /
 * tumpy.argsort.  Replaces the sort pallas_calls of
 *   tax.sort(operand, num_keys, is_stable, return_argsort, descending)
 *   -- tallax/_src/sort.py:768-929 (engine sort.py:414-571; key transforms
 *   utils.py:139-227); tumpy.sort/argsort -- tallax/tumpy.py:6-97.
 * Orders each row of `key` [rows, cols] (f32/bf16/int32; floats standardised:
 * NaN above +inf, -0 == +0) ascending, or descending, with ties by ascending
 * index (descending index when ties_descending).  With perm_in, sorts
 * key[row, perm_in[row, j]] with ties by position j and composes, so that
 * repeated calls give a stable multi-key (LSD) sort.  Outputs: perm_out
 * [rows, cols] int32 = source column of each sorted position; optional
 * key_out = the sorted keys decoded (f32 keys: f32; int32: int32; bf16: bf16
 * with NaN 0x7FFF, or f32 with NaN 0x7FFFFFFE, chosen by key_out_dtype);
 * optional aux / aux_out: a second key gathered by perm_out and decoded the
 * same way.  tallax_sort_rows takes rows of up to 16384 elements (one
 * workgroup sorts a row in LDS); tallax_sort_rows_ws takes any cols < 2^31
 * and uses `workspace` for longer rows (the reference's HBM substage route,
 * sort.py:574-758): at least tallax_sort_rows_workspace_size(rows, cols)
 * bytes, 0 for cols <= 16384, no initial contents needed.
 * ---------------------------------------------------------------------- */
int tallax_sort_rows(const void* key, int key_dtype, int64_t rows, int64_t cols, int descending,
                     int ties_descending, const int32_t* perm_in, int32_t* perm_out, void* key_out,
                     int key_out_dtype, const void* aux, int aux_dtype, void* aux_out, int aux_out_dtype,
                     tallax_stream_t stream);
size_t tallax_sort_rows_workspace_size(int64_t rows, int64_t cols);
/* The third and later keys of a multi-key sort (sort.py:912-919 decodes every
 * key operand): out[r, j] = key[r, perm[r, j]] standardised and decoded as
 * key_out is (out_dtype as for key_out).  perm [rows, cols] int32 from
 * tallax_sort_rows; a column outside the row gives 0. */
int tallax_gather_sort_key(const void* key, int key_dtype, int64_t rows, int64_t cols, const int32_t* perm,
                           void* out, int out_dtype, tallax_stream_t stream);
int tallax_sort_rows_ws(const void* key, int key_dtype, int64_t rows, int64_t cols, int descending,
                        int ties_descending, const int32_t* perm_in, int32_t* perm_out, void* key_out,
                        int key_out_dtype, const void* aux, int aux_dtype, void* aux_out, int aux_out_dtype,
                        void* workspace, size_t workspace_bytes, tallax_stream_t stream);

/* ------------------------------------------------------------------------
 * Prefill-scale softmax -> top-k -> cumsum -> top-p cutoff, fused (BASELINE
 * config 5).  Replaces the composition the reference runs for it:
 * jax.nn.softmax, tax.sort(probs, descending=True, return_argsort=True) cut
 * to k (tallax/_src/sort.py:768-929), tax.cumsum(axis=1)
 * (tallax/_src/cumsum.py:75-101) and sum(cumsum < p).
 * logits [rows, cols] f32 -> out_probs [rows, k] f32 (descending softmax
 * probabilities), out_idx [rows, k] int32 (the k largest logits, ties to the
 * lowest index), out_cumsum [rows, k] f32 (tile order of tax.cumsum),
 * out_cutoff [rows] int32 = #(cumsum < p).  1 <= k <= 2048, k <= cols.
 * Rows holding NaN or +inf give NaN probabilities, indices 0..k-1, cutoff 0.
 * ---------------------------------------------------------------------- */
int tallax_softmax_topk_cumsum(const float* logits, int64_t rows, int64_t cols, int k, float p, float* out_probs,
                               int32_t* out_idx, float* out_cumsum, int32_t* out_cutoff, tallax_stream_t stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* TALLAX_HIP_H_ */
