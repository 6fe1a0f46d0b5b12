/*
 * tallax_hip_testing.h -- test hooks of the MI355X tallax library.
 *
 * These entry points have NO counterpart in the reference: they expose the
 * device-side primitives the sampler is built from (float32 exp/log and the
 * Threefry-2x32 Gumbel noise) so that tests can compare them bit for bit with
 * the CPU oracle.  Conventions are those of tallax_hip.h.
 */
#ifndef TALLAX_HIP_TESTING_H_
#define TALLAX_HIP_TESTING_H_

#include <stddef.h>
#include <stdint.h>

#include "tallax_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* exp_out[i] = exp(x[i]), log_out[i] = log(x[i]) with the sampler's float32 routines. */
int tallax_testing_expf_logf(const float* x, float* exp_out, float* log_out, int64_t n,
                             tallax_stream_t stream);

/* bits_out[i] = x0 ^ x1 of threefry2x32((k0, k1), (0, counters[i])) and
 * gumbel_out[i] = -log(-log(max(tiny, unit(bits)*(1-tiny) + tiny))). */
int tallax_testing_gumbel(uint32_t k0, uint32_t k1, const uint32_t* counters, float* gumbel_out,
                          uint32_t* bits_out, int64_t n, tallax_stream_t stream);

/* out[64 * d + lane] = value of lane (lane ^ 2^d) for d = 0..5 and
 * out[384 + lane] = value of lane (63 - lane), as seen through the wave64
 * lane-exchange helpers of the kernels (DPP / v_permlane*_swap); out holds 448 words. */
int tallax_testing_lane_ops(uint32_t* out, tallax_stream_t stream);

/* Work split the selection entry points (tallax_topk, tallax_fused_topk_topp_sample)
 * choose for a [rows, cols] input of `dtype`: out[0] threads per workgroup,
 * out[1] 16-byte vectors per thread, out[2] workgroups (segments) per row,
 * out[3] vectors per segment.  Host only: no device work. */
int tallax_testing_select_plan(int64_t rows, int64_t cols, int dtype, int32_t* out);

/* tallax_top_dynamic_k with its path chosen by `path`: 0 (what
 * tallax_top_dynamic_k runs) settles rows from the exact kernel's per-segment
 * top-128 candidates where they suffice and scans the rest; 1 scans every
 * row.  Both give the same results; tests run both.  Other arguments as
 * tallax_top_dynamic_k; TALLAX_INVALID_ARGUMENT for another path. */
int tallax_testing_top_dynamic_k_path(const void* x, int dtype, int64_t rows, int64_t cols, const int32_t* k_rows,
                                      int max_k, int block_token, int num_bins, const int32_t* schedule,
                                      int num_steps, int guarantee_convergence, int has_replace,
                                      double replace_val, void* out_vals,
                                      int32_t* out_idx, int32_t* out_valid, int32_t* out_depths, float* out_cutoff,
                                      void* workspace, size_t workspace_bytes, tallax_stream_t stream, int path);

/* Reads nbytes of src with `width`-byte loads (4, 8 or 16; src aligned to it,
 * nbytes a multiple of it) and writes one word per workgroup to out (2048
 * words): the calibration launch for the FETCH_SIZE counter. */
int tallax_testing_read_bytes(const void* src, int64_t nbytes, int width, uint32_t* out, tallax_stream_t stream);

/* One LDS atomic add per lane of each wave on the counter of its digit
 * (digits[i] mod ndig, 1 <= ndig <= 256), 256 lanes per workgroup, nblocks
 * workgroups: out[i] = the counter's value before lane i's add.  The bf16
 * radix sort relies on these adds returning in ascending lane order. */
int tallax_testing_lds_atomic_order(const uint32_t* digits, int64_t nblocks, int ndig, uint32_t* out,
                                    tallax_stream_t stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* TALLAX_HIP_TESTING_H_ */
