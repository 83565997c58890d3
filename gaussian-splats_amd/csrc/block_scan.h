// Wave64 / 256-thread workgroup prefix sums used by the scan and radix kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace gs {

template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v) {
  const int lane = __lane_id();
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const T t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Exclusive prefix over a 256-thread block (4 waves); returns the block total
// through `total`.  `scratch` must hold 4 values and is reused after return.
template <typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T* scratch, T& total) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const T inc = wave_inclusive_scan(v);
  if (lane == 63) scratch[wid] = inc;
  __syncthreads();
  T before = 0;
  T sum = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const T s = scratch[w];
    if (w < wid) before += s;
    sum += s;
  }
  total = sum;
  __syncthreads();
  return inc - v + before;
}

}  // namespace gs
