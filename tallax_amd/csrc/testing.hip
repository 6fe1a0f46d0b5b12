// Test hooks: expose the device-side exp/log/Gumbel primitives so that the
// GPU test suite can pin them bit for bit against the numpy oracle, and a
// read kernel of known traffic for counter calibration.  These
// entry points have no counterpart in the reference.
#include "tallax_hip_testing.h"
#include "tx_common.h"
#include "tx_host.h"
#include "tx_math.h"

#include <type_traits>

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

// out[d * 64 + lane] = lane_xor(lane, 1 << d) for d = 0..5, out[6 * 64 + lane] = lane_rev(lane).
__global__ void lane_ops_kernel(uint32_t* out) {
  const uint32_t x = threadIdx.x;
  out[0 * 64 + x] = lane_xor(x, 1);
  out[1 * 64 + x] = lane_xor(x, 2);
  out[2 * 64 + x] = lane_xor(x, 4);
  out[3 * 64 + x] = lane_xor(x, 8);
  out[4 * 64 + x] = lane_xor(x, 16);
  out[5 * 64 + x] = lane_xor(x, 32);
  out[6 * 64 + x] = lane_rev(x);
}

}  // namespace tx

// Reads nbytes (a multiple of W) with W-byte loads, grid-stride, and writes
// one XOR of the words per workgroup: the counter calibration kernel (the
// FETCH_SIZE of a launch that reads a known number of bytes with loads of a
// known width).
namespace tx {

constexpr int kReadProbeBlocks = 2048;
template <int W>
__global__ __launch_bounds__(256) void read_probe_kernel(const void* src, int64_t nbytes, uint32_t* out) {
  using V = typename std::conditional<W == 16, uint4, typename std::conditional<W == 8, uint2, uint32_t>::type>::type;
  const V* p = (const V*)src;
  const int64_t n = nbytes / W;
  uint32_t acc = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const V v = p[i];
    if constexpr (W == 16) acc ^= v.x ^ v.y ^ v.z ^ v.w;
    else if constexpr (W == 8) acc ^= v.x ^ v.y;
    else acc ^= v;
  }
  acc = (uint32_t)wave_sum_i((int)acc);  // any combination: it only has to be written
  __shared__ uint32_t red[4];
  if (lane_id() == 0) red[threadIdx.x / kWave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

}  // namespace tx

// Every lane of a wave adds 1 to the LDS counter of its digit (digits[] mod
// ndig) in one atomic instruction; out[] gets the value before each add.
// Lane-ordered atomics give each lane the count of lower lanes with its digit.
__global__ __launch_bounds__(256) void lds_atomic_order_kernel(const uint32_t* digits, int ndig, uint32_t* out) {
  __shared__ uint32_t cnt[4][256];
  const int w = threadIdx.x / 64;
  for (int i = threadIdx.x; i < 4 * 256; i += 256) cnt[i / 256][i % 256] = 0u;
  __syncthreads();
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  out[e] = atomicAdd(&cnt[w][digits[e] % (uint32_t)ndig], 1u);
}

extern "C" {

int tallax_testing_lane_ops(uint32_t* out, hipStream_t stream) {
  if (!out) {
    tx::set_error("bad arguments");
    return tx::kInvalidArgument;
  }
  hipLaunchKernelGGL(tx::lane_ops_kernel, dim3(1), dim3(64), 0, stream, out);
  return tx::launch_status("tallax_testing_lane_ops");
}

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

int tallax_testing_read_bytes(const void* src, int64_t nbytes, int width, uint32_t* out, hipStream_t stream) {
  if ((width != 4 && width != 8 && width != 16) || nbytes <= 0 || nbytes % width || !src || !out ||
      ((uintptr_t)src % width)) {
    tx::set_error("bad arguments");
    return tx::kInvalidArgument;
  }
  const dim3 grid(tx::kReadProbeBlocks), block(256);
  if (width == 16) hipLaunchKernelGGL(tx::read_probe_kernel<16>, grid, block, 0, stream, src, nbytes, out);
  else if (width == 8) hipLaunchKernelGGL(tx::read_probe_kernel<8>, grid, block, 0, stream, src, nbytes, out);
  else hipLaunchKernelGGL(tx::read_probe_kernel<4>, grid, block, 0, stream, src, nbytes, out);
  return tx::launch_status("tallax_testing_read_bytes");
}


int tallax_testing_lds_atomic_order(const uint32_t* digits, int64_t nblocks, int ndig, uint32_t* out,
                                    hipStream_t stream) {
  if (!digits || !out || nblocks <= 0 || nblocks > 65535 || ndig < 1 || ndig > 256) {
    tx::set_error("lds_atomic_order: bad arguments");
    return tx::kInvalidArgument;
  }
  hipLaunchKernelGGL(lds_atomic_order_kernel, dim3((unsigned)nblocks), dim3(256), 0, stream, digits, ndig, out);
  return tx::launch_status("tallax_testing_lds_atomic_order");
}

}  // extern "C"
