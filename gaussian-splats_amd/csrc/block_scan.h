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

// 32-bit DPP read of another lane (lanes outside row_mask, or whose source is
// out of range when ZERO, read 0).
template <int CTRL, int ROW_MASK, bool ZERO>
__device__ __forceinline__ uint32_t dpp_read(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), CTRL, ROW_MASK, 0xF, ZERO));
}

// Inclusive scan of a 32-bit value over the wave for an operation with
// identity 0 (sum, or max of unsigned values): Hillis-Steele inside each row
// of 16 lanes (row_shr 1, 2, 4, 8), then row_bcast:15 into rows 1 and 3 and
// row_bcast:31 into rows 2 and 3.  Six DPP operations instead of six
// ds_bpermute round trips.  Needs a full EXEC.
template <typename Op>
__device__ __forceinline__ uint32_t wave_inclusive_dpp(uint32_t v, Op op) {
  v = op(v, dpp_read<0x111, 0xF, true>(v));
  v = op(v, dpp_read<0x112, 0xF, true>(v));
  v = op(v, dpp_read<0x114, 0xF, true>(v));
  v = op(v, dpp_read<0x118, 0xF, true>(v));
  v = op(v, dpp_read<0x142, 0xA, false>(v));
  v = op(v, dpp_read<0x143, 0xC, false>(v));
  return v;
}

struct AddOp {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a + b; }
};
struct MaxOp {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; }
};

template <>
__device__ __forceinline__ uint32_t wave_inclusive_scan<uint32_t>(uint32_t v) {
  return wave_inclusive_dpp(v, AddOp{});
}

template <>
__device__ __forceinline__ int32_t wave_inclusive_scan<int32_t>(int32_t v) {
  return int32_t(wave_inclusive_dpp(uint32_t(v), AddOp{}));
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Exclusive prefix over a block of NW waves; returns the block total through
// `total`.  `scratch` must hold NW values and is reused after return.
template <int NW, typename T>
__device__ __forceinline__ T block_exclusive_scan_waves(T v, T* scratch, T& total) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const T inc = wave_inclusive_scan(v);
  if (lane == 63) scratch[wid] = inc;
  __syncthreads();
  T before = 0;
  T sum = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const T s = scratch[w];
    if (w < wid) before += s;
    sum += s;
  }
  total = sum;
  __syncthreads();
  return inc - v + before;
}

// Four-wave workgroups (256 threads).
template <typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T* scratch, T& total) {
  return block_exclusive_scan_waves<4>(v, scratch, total);
}

}  // namespace gs
