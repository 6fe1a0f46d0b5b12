// Workgroup-wide bitonic sort of P = 2^m records held E per thread.
//
// Thread t holds records [t*E, (t+1)*E) in registers (P = blockDim.x * E).
// Compare-exchange partners at stride s are exchanged inside the thread
// (s < E), across lanes with DPP / v_permlane*_swap (s < 64 E), or through LDS
// (larger strides, one store / barrier / load / barrier round each).
#pragma once
#include "tx_common.h"
#include "tx_wave_sort.h"

namespace tx {

template <typename R>
__device__ __forceinline__ void cx_pair(R& a, R& b, bool asc) {
  const bool sw = (a > b) == asc;
  const R lo = sw ? b : a;
  const R hi = sw ? a : b;
  a = lo;
  b = hi;
}

// one stage at a stride S < E: pairs inside the thread's registers
template <typename R, int E, int S>
__device__ __forceinline__ void bsort_intra_stage(R v[E], int size, int t, bool desc) {
  if (S >= E) return;
#pragma unroll
  for (int r = 0; r < E; ++r) {
    if ((r & S) == 0) {
      const int i = t * E + r;
      cx_pair(v[r], v[r | S], ((i & size) == 0) != desc);
    }
  }
}

// one cross-lane stage at lane distance d (1..32)
template <typename R, int E>
__device__ __forceinline__ void bsort_lane_stage(R v[E], int d, int size, int t, bool desc) {
  const int l = lane_id();
  const bool lower = (l & d) == 0;
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int i = t * E + r;
    const bool asc = ((i & size) == 0) != desc;
    R o;
    switch (d) {
      case 1: o = lane_xor_c(v[r], 1); break;
      case 2: o = lane_xor_c(v[r], 2); break;
      case 4: o = lane_xor_c(v[r], 4); break;
      case 8: o = lane_xor_c(v[r], 8); break;
      case 16: o = lane_xor_c(v[r], 16); break;
      default: o = lane_xor_c(v[r], 32); break;
    }
    v[r] = cx(v[r], o, lower != asc);  // lower element keeps the min of an ascending pair
  }
}

// Sort the P = blockDim.x * E records ascending (or descending).  `lds` holds
// P records.  Every thread of the workgroup must call it.
template <typename R, int E>
__device__ __forceinline__ void block_bitonic_sort(R v[E], R* lds, int P, bool desc) {
  const int t = threadIdx.x;
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride >= 1; stride >>= 1) {
      if (stride < E) {
        switch (stride) {
          case 1: bsort_intra_stage<R, E, 1>(v, size, t, desc); break;
          case 2: bsort_intra_stage<R, E, 2>(v, size, t, desc); break;
          case 4: bsort_intra_stage<R, E, 4>(v, size, t, desc); break;
          default: bsort_intra_stage<R, E, 8>(v, size, t, desc); break;
        }
      } else if (stride < kWave * E) {
        bsort_lane_stage<R, E>(v, stride / E, size, t, desc);
      } else {
#pragma unroll
        for (int r = 0; r < E; ++r) lds[t * E + r] = v[r];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < E; ++r) {
          const int i = t * E + r;
          const R o = lds[i ^ stride];
          const bool asc = ((i & size) == 0) != desc;
          const bool lower = (i & stride) == 0;
          v[r] = cx(v[r], o, lower != asc);
        }
        __syncthreads();
      }
    }
  }
}

// The same network with P known at compile time.  Each (size, stride) stage
// is its own template instance, reached by compile-time recursion rather than
// by unrolling the nested size / stride loops: the loops' trip counts grow
// as log^2 P and the unroller gives up on them for P = 16384, which left the
// register array indexed at run time (VGPR indexing or scratch).  Here every
// record index is a constant.
template <typename R, int E, int SIZE, int STRIDE, bool DESC>
__device__ __forceinline__ void bitonic_stage_c(R (&v)[E], R* lds) {
  const int t = threadIdx.x;
  if constexpr (STRIDE < E) {
#pragma unroll
    for (int r = 0; r < E; ++r) {
      if ((r & STRIDE) == 0) {
        const int i = t * E + r;
        cx_pair(v[r], v[r | STRIDE], ((i & SIZE) == 0) != DESC);
      }
    }
  } else if constexpr (STRIDE < kWave * E) {
    bsort_lane_stage<R, E>(v, STRIDE / E, SIZE, t, DESC);
  } else {
#pragma unroll
    for (int r = 0; r < E; ++r) lds[t * E + r] = v[r];
    __syncthreads();
#pragma unroll
    for (int r = 0; r < E; ++r) {
      const int i = t * E + r;
      const R o = lds[i ^ STRIDE];
      const bool asc = ((i & SIZE) == 0) != DESC;
      const bool lower = (i & STRIDE) == 0;
      v[r] = cx(v[r], o, lower != asc);
    }
    __syncthreads();
  }
}

template <typename R, int E, int P, int SIZE, int STRIDE, bool DESC>
__device__ __forceinline__ void bitonic_from_c(R (&v)[E], R* lds) {
  bitonic_stage_c<R, E, SIZE, STRIDE, DESC>(v, lds);
  if constexpr (STRIDE > 1) {
    bitonic_from_c<R, E, P, SIZE, STRIDE / 2, DESC>(v, lds);
  } else if constexpr (SIZE < P) {
    bitonic_from_c<R, E, P, SIZE * 2, SIZE, DESC>(v, lds);
  }
}

template <typename R, int E, int P, bool DESC>
__device__ __forceinline__ void block_bitonic_sort_c(R (&v)[E], R* lds) {
  static_assert((P & (P - 1)) == 0 && P >= 2 && P % E == 0, "P: a power of two, E records per thread");
  bitonic_from_c<R, E, P, 2, 1, DESC>(v, lds);
}

}  // namespace tx
