// Test hooks: expose the device-side exp/log/Gumbel primitives so that the
// GPU test suite can pin them bit for bit against the numpy oracle.  These
// entry points have no counterpart in the reference.
#include "tallax_hip_testing.h"
#include "tx_common.h"
#include "tx_host.h"
#include "tx_math.h"

namespace tx {

__global__ void math_probe_kernel(const float* x, float* e, float* l, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    e[i] = tx_expf(x[i]);
    l[i] = tx_logf(x[i]);
  }
}

__global__ void gumbel_probe_kernel(uint32_t k0, uint32_t k1, const uint32_t* ctr, float* g,
                                    uint32_t* bits, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    uint32_t o0, o1;
    threefry2x32(k0, k1, 0u, ctr[i], o0, o1);
    bits[i] = o0 ^ o1;
    g[i] = gumbel_from_bits(o0 ^ o1);
  }
}

}  // namespace tx

extern "C" {

int tallax_testing_expf_logf(const float* x, float* exp_out, float* log_out, int64_t n,
                             hipStream_t stream) {
  if (n < 0 || (n > 0 && (!x || !exp_out || !log_out))) {
    tx::set_error("bad arguments");
    return tx::kInvalidArgument;
  }
  if (n == 0) return tx::kOk;
  const unsigned blocks = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(tx::math_probe_kernel, dim3(blocks), dim3(256), 0, stream, x, exp_out, log_out, n);
  return tx::launch_status("tallax_testing_expf_logf");
}

int tallax_testing_gumbel(uint32_t k0, uint32_t k1, const uint32_t* counters, float* gumbel_out,
                          uint32_t* bits_out, int64_t n, hipStream_t stream) {
  if (n < 0 || (n > 0 && (!counters || !gumbel_out || !bits_out))) {
    tx::set_error("bad arguments");
    return tx::kInvalidArgument;
  }
  if (n == 0) return tx::kOk;
  const unsigned blocks = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(tx::gumbel_probe_kernel, dim3(blocks), dim3(256), 0, stream, k0, k1, counters,
                     gumbel_out, bits_out, n);
  return tx::launch_status("tallax_testing_gumbel");
}

}  // extern "C"
