// Tile binning: count scan, load-balanced intersection emission, stable LSD
// radix sort and per-tile ranges.
//
// Reference path being replaced: kernels/rasterize/intersections.py:10-88
// (scan with a host read of the total, serial per-Gaussian emission, a full
// 64-bit torch.sort and bincount/cumsum ranges) and torch.py:254-287.
//
// Two orderings are offered, both bit-identical to a stable sort of the
// reference keys (tile_id << 32 | depth bits) emitted in Gaussian order:
//  * reference format: emit 64-bit keys in Gaussian order, sort over
//    32 + ceil(log2 T) bits (gs_emit_intersections / gs_sort_intersections);
//  * fused format: sort the N Gaussians by (depth bits, index) first, emit in
//    that order with 32-bit tile keys, then sort over ceil(log2 T) bits only
//    (gs_bin_gaussians / gs_emit_tiles / gs_sort_tiles).  A stable sort by tile
//    of a depth-ordered stream leaves each tile ordered by (depth bits, index),
//    exactly the order the 64-bit stable sort produces, while moving
//    4+4 bytes per intersection per pass over 2 passes instead of 8+4 bytes
//    over 6.
#include "block_scan.h"
#include "common.h"

namespace gs {
namespace {

constexpr int kBlock = 256;
constexpr int kItems = 16;
constexpr int kTileItems = kBlock * kItems;  // elements per workgroup

// ---------------------------------------------------------------------------
// Device-wide exclusive scan (reduce -> scan of block sums -> downsweep).
// value(i) = in[order ? order[i] : i]; out[n] receives the total when
// write_total is set.
// ---------------------------------------------------------------------------
template <typename In, typename Out>
__global__ __launch_bounds__(kBlock) void scan_reduce_kernel(const In* __restrict__ in,
                                                             const int32_t* __restrict__ order,
                                                             int64_t n, Out* __restrict__ sums) {
  __shared__ Out scratch[4];
  const int64_t base = int64_t(blockIdx.x) * kTileItems;
  Out s = 0;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int64_t idx = base + i * kBlock + threadIdx.x;
    if (idx < n) s += Out(in[order ? order[idx] : idx]);
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) sums[blockIdx.x] = scratch[0] + scratch[1] + scratch[2] + scratch[3];
}

// One workgroup scans the block sums in place, chunk by chunk.
template <typename Out>
__global__ __launch_bounds__(kBlock) void scan_sums_kernel(Out* __restrict__ sums, int64_t nb,
                                                           Out* __restrict__ total_out) {
  __shared__ Out scratch[4];
  Out carry = 0;
  for (int64_t chunk = 0; chunk < nb; chunk += kBlock) {
    const int64_t idx = chunk + threadIdx.x;
    const Out v = idx < nb ? sums[idx] : Out(0);
    Out total;
    const Out ex = block_exclusive_scan(v, scratch, total);
    if (idx < nb) sums[idx] = carry + ex;
    carry += total;
  }
  if (total_out && threadIdx.x == 0) *total_out = carry;
}

template <typename In, typename Out>
__global__ __launch_bounds__(kBlock) void scan_down_kernel(const In* __restrict__ in,
                                                           const int32_t* __restrict__ order,
                                                           int64_t n,
                                                           const Out* __restrict__ block_offsets,
                                                           Out* __restrict__ out) {
  __shared__ Out scratch[4];
  const int64_t base = int64_t(blockIdx.x) * kTileItems;
  Out carry = block_offsets[blockIdx.x];
  for (int i = 0; i < kItems; ++i) {
    const int64_t idx = base + i * kBlock + threadIdx.x;
    const Out v = idx < n ? Out(in[order ? order[idx] : idx]) : Out(0);
    Out total;
    const Out ex = block_exclusive_scan(v, scratch, total);
    if (idx < n) out[idx] = carry + ex;
    carry += total;
  }
}

template <typename T>
__global__ void fill_kernel(T* p, int64_t n, T value) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = value;
}

template <typename Out>
size_t scan_ws_bytes(int64_t n) {
  const int64_t nb = ceil_div(n, kTileItems);
  return align_up(size_t(nb + 1) * sizeof(Out));
}

// out[0..n) = exclusive prefix of value(i); out[n] = total when write_total.
template <typename In, typename Out>
int device_exclusive_scan(const In* in, const int32_t* order, int64_t n, Out* out,
                          bool write_total, void* ws, hipStream_t s) {
  if (n == 0) {
    if (write_total) fill_kernel<Out><<<1, 64, 0, s>>>(out, 1, Out(0));
    return check_launch("scan(empty)");
  }
  const int64_t nb = ceil_div(n, kTileItems);
  Out* sums = static_cast<Out*>(ws);
  scan_reduce_kernel<In, Out><<<unsigned(nb), kBlock, 0, s>>>(in, order, n, sums);
  scan_sums_kernel<Out><<<1, kBlock, 0, s>>>(sums, nb, write_total ? out + n : nullptr);
  scan_down_kernel<In, Out><<<unsigned(nb), kBlock, 0, s>>>(in, order, n, sums, out);
  return check_launch("scan");
}

// ---------------------------------------------------------------------------
// Stable LSD radix sort of (key, u32 value) pairs.
//
// Per pass: histogram (per-wave LDS counters) -> digit-major exclusive scan of
// the [digit][workgroup] counts -> scatter.  The scatter ranks each element
// within its wave by matching digits with ballots (stable: lane order inside
// an iteration, iterations in input order), combines the four wave segments of
// the workgroup through LDS, reorders the 4096-element tile in LDS by digit and
// writes it out with consecutive lanes on consecutive addresses.
// ---------------------------------------------------------------------------
template <typename K, int BITS>
__global__ __launch_bounds__(kBlock) void radix_hist_kernel(const K* __restrict__ keys, int64_t n,
                                                            int shift, uint32_t* __restrict__ hist,
                                                            int nblocks) {
  constexpr int D = 1 << BITS;
  __shared__ uint32_t h[4][D];
  const int wid = threadIdx.x >> 6;
  for (int d = threadIdx.x; d < 4 * D; d += kBlock) (&h[0][0])[d] = 0;
  __syncthreads();
  const int64_t base = int64_t(blockIdx.x) * kTileItems;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int64_t idx = base + i * kBlock + threadIdx.x;
    if (idx < n) {
      const uint32_t d = uint32_t(keys[idx] >> shift) & (D - 1);
      atomicAdd(&h[wid][d], 1u);
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += kBlock)
    hist[int64_t(d) * nblocks + blockIdx.x] = h[0][d] + h[1][d] + h[2][d] + h[3][d];
}

template <typename K, int BITS>
__global__ __launch_bounds__(kBlock) void radix_scatter_kernel(
    const K* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, K* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out, int64_t n, int shift, const uint32_t* __restrict__ offsets,
    int nblocks) {
  constexpr int D = 1 << BITS;
  constexpr int kSeg = kTileItems / 4;  // contiguous elements per wave
  __shared__ uint32_t cnt[4][D];
  __shared__ uint32_t dstart[D];
  __shared__ uint32_t gofs[D];
  __shared__ uint32_t scratch[4];
  __shared__ K skeys[kTileItems];
  __shared__ uint32_t svals[kTileItems];

  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  for (int d = threadIdx.x; d < 4 * D; d += kBlock) (&cnt[0][0])[d] = 0;
  __syncthreads();

  const int64_t base = int64_t(blockIdx.x) * kTileItems;
  const int64_t seg = base + int64_t(wid) * kSeg;
  const uint64_t below = lanemask_lt();
  volatile uint32_t* wcnt = cnt[wid];

  K key[kItems];
  uint32_t val[kItems];
  uint32_t rank[kItems];
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int64_t idx = seg + i * 64 + lane;
    const bool valid = idx < n;
    key[i] = valid ? keys_in[idx] : K(0);
    val[i] = valid ? (vals_in ? vals_in[idx] : uint32_t(idx)) : 0u;
    const uint32_t d = uint32_t(key[i] >> shift) & (D - 1);
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < BITS; ++b) {
      const uint64_t ones = __ballot((d >> b) & 1u);
      peers &= ((d >> b) & 1u) ? ones : ~ones;
    }
    const uint32_t before = uint32_t(__popcll(peers & below));
    uint32_t c = 0;
    if (valid) c = wcnt[d];
    if (valid && before == 0) wcnt[d] = c + uint32_t(__popcll(peers));
    rank[i] = c + before;
  }
  __syncthreads();

  // Per digit: exclusive prefix over the four wave segments, block-local
  // digit start, and the global offset of this workgroup's digit bucket.
  uint32_t tot = 0;
  if (threadIdx.x < D) {
    const uint32_t c0 = cnt[0][threadIdx.x], c1 = cnt[1][threadIdx.x];
    const uint32_t c2 = cnt[2][threadIdx.x], c3 = cnt[3][threadIdx.x];
    cnt[0][threadIdx.x] = 0;
    cnt[1][threadIdx.x] = c0;
    cnt[2][threadIdx.x] = c0 + c1;
    cnt[3][threadIdx.x] = c0 + c1 + c2;
    tot = c0 + c1 + c2 + c3;
    gofs[threadIdx.x] = offsets[int64_t(threadIdx.x) * nblocks + blockIdx.x];
  }
  uint32_t all;
  const uint32_t start = block_exclusive_scan(tot, scratch, all);
  if (threadIdx.x < D) dstart[threadIdx.x] = start;
  __syncthreads();

#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int64_t idx = seg + i * 64 + lane;
    if (idx < n) {
      const uint32_t d = uint32_t(key[i] >> shift) & (D - 1);
      const uint32_t pos = dstart[d] + cnt[wid][d] + rank[i];
      skeys[pos] = key[i];
      svals[pos] = val[i];
    }
  }
  __syncthreads();

  const int nvalid = int(min(int64_t(kTileItems), n - base));
  for (int j = threadIdx.x; j < nvalid; j += kBlock) {
    const K k = skeys[j];
    const uint32_t d = uint32_t(k >> shift) & (D - 1);
    const int64_t o = int64_t(gofs[d]) + (j - int(dstart[d]));
    keys_out[o] = k;
    vals_out[o] = svals[j];
  }
}

template <typename K, int BITS>
void launch_pass(const K* kin, const uint32_t* vin, K* kout, uint32_t* vout, int64_t n, int shift,
                 uint32_t* hist, void* scan_ws, int nblocks, hipStream_t s) {
  radix_hist_kernel<K, BITS><<<unsigned(nblocks), kBlock, 0, s>>>(kin, n, shift, hist, nblocks);
  device_exclusive_scan<uint32_t, uint32_t>(hist, nullptr, int64_t(nblocks) << BITS, hist, false,
                                            scan_ws, s);
  radix_scatter_kernel<K, BITS><<<unsigned(nblocks), kBlock, 0, s>>>(kin, vin, kout, vout, n, shift,
                                                                     hist, nblocks);
}

template <typename K>
void dispatch_pass(int bits, const K* kin, const uint32_t* vin, K* kout, uint32_t* vout, int64_t n,
                   int shift, uint32_t* hist, void* scan_ws, int nblocks, hipStream_t s) {
  switch (bits) {
    case 1: launch_pass<K, 1>(kin, vin, kout, vout, n, shift, hist, scan_ws, nblocks, s); break;
    case 2: launch_pass<K, 2>(kin, vin, kout, vout, n, shift, hist, scan_ws, nblocks, s); break;
    case 3: launch_pass<K, 3>(kin, vin, kout, vout, n, shift, hist, scan_ws, nblocks, s); break;
    case 4: launch_pass<K, 4>(kin, vin, kout, vout, n, shift, hist, scan_ws, nblocks, s); break;
    case 5: launch_pass<K, 5>(kin, vin, kout, vout, n, shift, hist, scan_ws, nblocks, s); break;
    case 6: launch_pass<K, 6>(kin, vin, kout, vout, n, shift, hist, scan_ws, nblocks, s); break;
    case 7: launch_pass<K, 7>(kin, vin, kout, vout, n, shift, hist, scan_ws, nblocks, s); break;
    default: launch_pass<K, 8>(kin, vin, kout, vout, n, shift, hist, scan_ws, nblocks, s); break;
  }
}

int bits_for(int64_t count) {  // ceil(log2(count)), 0 for count <= 1
  int b = 0;
  while ((int64_t(1) << b) < count) ++b;
  return b;
}

// Workspace layout of one sort: [keys_alt | vals_a | vals_b | hist | scan].
template <typename K>
size_t sort_ws_bytes(int64_t n) {
  const int64_t nblocks = ceil_div(n, kTileItems);
  return align_up(size_t(n) * sizeof(K)) + 2 * align_up(size_t(n) * 4) +
         align_up(size_t(nblocks) * 256 * 4) + scan_ws_bytes<uint32_t>(nblocks * 256);
}

// Sorts (keys, vals) on bits [0, end_bit); vals == nullptr means vals[i] = i.
// The sorted values land in vals_final; *keys_final points at the sorted keys
// (either `keys` or the workspace copy).  keys and vals are clobbered.
template <typename K>
int radix_sort(K* keys, const uint32_t* vals, int64_t n, int end_bit, uint32_t* vals_final,
               K** keys_final, void* ws, size_t ws_bytes, hipStream_t s) {
  GS_REQUIRE(ws_bytes >= sort_ws_bytes<K>(n), GS_ERR_WORKSPACE,
             "sort workspace too small (%zu < %zu)", ws_bytes, sort_ws_bytes<K>(n));
  GS_REQUIRE(n < (int64_t(1) << 32) - kTileItems, GS_ERR_OVERFLOW,
             "too many elements to sort (%lld)", (long long)n);
  char* p = static_cast<char*>(ws);
  K* keys_alt = reinterpret_cast<K*>(p);
  p += align_up(size_t(n) * sizeof(K));
  uint32_t* vbuf[2];
  vbuf[0] = reinterpret_cast<uint32_t*>(p);
  p += align_up(size_t(n) * 4);
  vbuf[1] = reinterpret_cast<uint32_t*>(p);
  p += align_up(size_t(n) * 4);
  const int nblocks = int(ceil_div(n, kTileItems));
  uint32_t* hist = reinterpret_cast<uint32_t*>(p);
  p += align_up(size_t(nblocks) * 256 * 4);
  void* scan_ws = p;

  K* kbuf[2] = {keys_alt, keys};
  if (n == 0) {
    *keys_final = keys;
    return GS_OK;
  }
  const int passes = end_bit <= 0 ? 1 : int(ceil_div(end_bit, 8));
  int shift = 0;
  const K* kin = keys;
  const uint32_t* vin = vals;
  for (int pass = 0; pass < passes; ++pass) {
    const int remaining = end_bit - shift;
    const int bits = end_bit <= 0 ? 1 : int(ceil_div(remaining, passes - pass));
    K* kout = kbuf[pass & 1];
    uint32_t* vout = (pass == passes - 1) ? vals_final : vbuf[pass & 1];
    dispatch_pass<K>(bits, kin, vin, kout, vout, n, shift, hist, scan_ws, nblocks, s);
    kin = kout;
    vin = vout;
    shift += bits;
  }
  *keys_final = const_cast<K*>(kin);
  return check_launch("radix_sort");
}

// ---------------------------------------------------------------------------
// Per-tile half-open ranges by binary search on the sorted tile ids.
// Empty tiles get [p, p) with p the number of intersections of lower tiles,
// as bincount + cumsum produce (intersections.py:84-88).
// ---------------------------------------------------------------------------
template <typename K, int SHIFT>
__global__ __launch_bounds__(256) void ranges_kernel(const K* __restrict__ keys, int64_t n,
                                                     int num_tiles, int64_t* __restrict__ ranges) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= num_tiles) return;
  auto lower = [&](uint64_t target) {
    int64_t lo = 0, hi = n;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if ((uint64_t(keys[mid]) >> SHIFT) < target) lo = mid + 1;
      else hi = mid;
    }
    return lo;
  };
  ranges[2 * t] = lower(uint64_t(t));
  ranges[2 * t + 1] = lower(uint64_t(t) + 1);
}

// ---------------------------------------------------------------------------
// Load-balanced emission.  Each wave owns a fixed chunk of kEmitChunk
// consecutive output slots [c0, c1).  It finds the Gaussian owning slot c0
// with a 64-ary search over the offsets (4 ballot rounds for 1M Gaussians),
// then walks windows of 64 consecutive positions p (Gaussian p, or the p-th
// Gaussian in depth order); inside a window the owner of slot e is found by a
// 6-step binary search over the window's offsets in LDS.  Work per wave is
// bounded by the chunk, so a Gaussian covering thousands of tiles (or a run of
// them, as the nearest Gaussians are after the depth sort) is spread over
// many waves.
// ---------------------------------------------------------------------------
constexpr int kEmitChunk = 2048;

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// local / w for 0 <= local, 1 <= w, via a float reciprocal and one correction.
__device__ __forceinline__ int div_small(int local, int w, int& rem) {
  int q;
  if (local < (1 << 22)) {
    q = int(float(local) * __builtin_amdgcn_rcpf(float(w)));
    int r = local - q * w;
    if (r < 0) {
      --q;
      r += w;
    } else if (r >= w) {
      ++q;
      r -= w;
    }
    rem = r;
  } else {
    q = local / w;
    rem = local - q * w;
  }
  return q;
}

template <bool REF_KEYS>
__global__ __launch_bounds__(kBlock) void emit_kernel(
    const int4* __restrict__ bounds, const int32_t* __restrict__ order,
    const float* __restrict__ depths, int64_t depth_stride, const int64_t* __restrict__ offsets,
    int64_t n, int64_t total, int tiles_w, void* __restrict__ keys_out,
    int32_t* __restrict__ ids_out) {
  __shared__ int64_t s_off[4][65];
  __shared__ int s_x0[4][64];
  __shared__ int s_w[4][64];
  __shared__ int s_y0[4][64];
  __shared__ uint32_t s_lo[4][64];
  __shared__ int s_id[4][64];

  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int64_t c0 = (int64_t(blockIdx.x) * 4 + wid) * kEmitChunk;
  if (c0 >= total) return;  // no workgroup barrier below
  const int64_t c1 = min(total, c0 + kEmitChunk);

  // Largest p < n with offsets[p] <= c0 (its count is > 0 because c0 < total).
  int64_t lo = 0, hi = n - 1;
  while (lo < hi) {
    const int64_t step = (hi - lo + 63) / 64;
    const int64_t q = min(lo + (lane + 1) * step, hi);
    const uint64_t m = __ballot(offsets[q] <= c0);
    const int cnt = __popcll(m);
    if (cnt == 0) {
      hi = lo + step - 1;
    } else {
      const int64_t new_lo = min(lo + cnt * step, hi);
      if (cnt < 64) hi = min(lo + (cnt + 1) * step - 1, hi);
      lo = new_lo;
    }
  }

  int64_t p = lo;
  int64_t e_begin = c0;
  while (e_begin < c1) {
    const int64_t pp = p + lane;
    if (pp < n) {
      const int g = order ? order[pp] : int(pp);
      const int4 b = bounds[g];
      s_off[wid][lane] = offsets[pp];
      s_x0[wid][lane] = b.x;
      s_w[wid][lane] = max(b.y - b.x, 1);
      s_y0[wid][lane] = b.z;
      s_id[wid][lane] = g;
      s_lo[wid][lane] = REF_KEYS ? __float_as_uint(depths[int64_t(g) * depth_stride]) : 0u;
    } else {
      s_off[wid][lane] = total;
      s_w[wid][lane] = 1;
    }
    if (lane == 0) s_off[wid][64] = offsets[min(p + 64, n)];
    wave_sync();
    const int64_t w_end = min(c1, s_off[wid][64]);
    for (int64_t e = e_begin + lane; e < w_end; e += 64) {
      int j = 0;
#pragma unroll
      for (int step = 32; step > 0; step >>= 1)
        if (s_off[wid][j + step] <= e) j += step;
      const int local = int(e - s_off[wid][j]);
      int col;
      const int row = div_small(local, s_w[wid][j], col);
      const uint32_t tile = uint32_t((s_y0[wid][j] + row) * tiles_w + s_x0[wid][j] + col);
      if (REF_KEYS) {
        static_cast<uint64_t*>(keys_out)[e] = (uint64_t(tile) << 32) | uint64_t(s_lo[wid][j]);
      } else {
        static_cast<uint32_t*>(keys_out)[e] = tile;
      }
      ids_out[e] = s_id[wid][j];
    }
    e_begin = max(e_begin, w_end);
    p += 64;
    wave_sync();
  }
}

unsigned emit_blocks(int64_t total) { return unsigned(ceil_div(total, int64_t(kEmitChunk) * 4)); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" {

GS_API size_t gs_scan_workspace_bytes(int64_t n) { return scan_ws_bytes<int64_t>(n < 0 ? 0 : n); }

GS_API int gs_scan_counts(const int32_t* counts, int64_t n, int64_t* offsets, void* workspace,
                          size_t workspace_bytes, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0 && offsets && (n == 0 || counts), GS_ERR_INVALID_ARGUMENT,
             "invalid scan arguments");
  GS_REQUIRE(workspace_bytes >= scan_ws_bytes<int64_t>(n) && (n == 0 || workspace),
             GS_ERR_WORKSPACE, "scan workspace too small");
  return device_exclusive_scan<int32_t, int64_t>(counts, nullptr, n, offsets, true, workspace,
                                                 as_stream(stream));
}

GS_API int gs_emit_intersections(const int32_t* bounds, const float* depths, int64_t depth_stride,
                                 const int64_t* offsets, int64_t n, int64_t total, int32_t tiles_w,
                                 int64_t* keys, int32_t* gaussian_ids, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0 && total >= 0 && tiles_w > 0, GS_ERR_INVALID_ARGUMENT,
             "invalid emit arguments");
  if (n == 0 || total == 0) return GS_OK;
  GS_REQUIRE(bounds && depths && offsets && keys && gaussian_ids && aligned16(bounds),
             GS_ERR_INVALID_ARGUMENT, "null or misaligned pointer");
  emit_kernel<true><<<emit_blocks(total), kBlock, 0, as_stream(stream)>>>(
      reinterpret_cast<const int4*>(bounds), nullptr, depths, depth_stride, offsets, n, total,
      tiles_w, keys, gaussian_ids);
  return check_launch("emit_intersections");
}

GS_API size_t gs_sort_workspace_bytes(int64_t total, int32_t num_tiles) {
  (void)num_tiles;
  if (total < 0) total = 0;
  return sort_ws_bytes<uint64_t>(total);
}

GS_API int gs_sort_intersections(int64_t* keys, int32_t* gaussian_ids, int64_t total,
                                 int32_t num_tiles, int32_t* sorted_ids, int64_t* ranges,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  GS_REQUIRE(total >= 0 && num_tiles > 0 && ranges, GS_ERR_INVALID_ARGUMENT,
             "invalid sort arguments");
  hipStream_t s = as_stream(stream);
  uint64_t* sorted_keys = reinterpret_cast<uint64_t*>(keys);
  if (total > 0) {
    GS_REQUIRE(keys && gaussian_ids && sorted_ids, GS_ERR_INVALID_ARGUMENT, "null pointer");
    GS_TRY(radix_sort<uint64_t>(reinterpret_cast<uint64_t*>(keys),
                                reinterpret_cast<const uint32_t*>(gaussian_ids), total,
                                32 + bits_for(num_tiles), reinterpret_cast<uint32_t*>(sorted_ids),
                                &sorted_keys, workspace, workspace_bytes, s));
  }
  ranges_kernel<uint64_t, 32><<<unsigned(ceil_div(num_tiles, 256)), 256, 0, s>>>(
      sorted_keys, total, num_tiles, ranges);
  return check_launch("sort_intersections");
}

GS_API size_t gs_bin_workspace_bytes(int64_t n) {
  if (n < 0) n = 0;
  return sort_ws_bytes<uint32_t>(n) + scan_ws_bytes<int64_t>(n);
}

GS_API int gs_bin_gaussians(uint32_t* depth_keys, const int32_t* counts, int64_t n,
                            int32_t* order, int64_t* offsets, void* workspace,
                            size_t workspace_bytes, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0 && offsets, GS_ERR_INVALID_ARGUMENT, "invalid binning arguments");
  GS_REQUIRE(workspace_bytes >= gs_bin_workspace_bytes(n), GS_ERR_WORKSPACE,
             "binning workspace too small");
  hipStream_t s = as_stream(stream);
  if (n == 0) return device_exclusive_scan<int32_t, int64_t>(counts, nullptr, 0, offsets, true,
                                                             workspace, s);
  GS_REQUIRE(depth_keys && counts && order, GS_ERR_INVALID_ARGUMENT, "null pointer");
  // depth_keys is used as a ping-pong buffer by the sort and is consumed.
  const size_t sort_bytes = sort_ws_bytes<uint32_t>(n);
  char* ws = static_cast<char*>(workspace);
  uint32_t* sorted_keys = nullptr;
  GS_TRY(radix_sort<uint32_t>(depth_keys, nullptr, n, 32, reinterpret_cast<uint32_t*>(order),
                              &sorted_keys, ws, sort_bytes, s));
  return device_exclusive_scan<int32_t, int64_t>(counts, order, n, offsets, true,
                                                 ws + sort_bytes, s);
}

GS_API int gs_emit_tiles(const int32_t* bounds, const int32_t* order, const int64_t* offsets,
                         int64_t n, int64_t total, int32_t tiles_w, uint32_t* tile_keys,
                         int32_t* gaussian_ids, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0 && total >= 0 && tiles_w > 0, GS_ERR_INVALID_ARGUMENT,
             "invalid emit arguments");
  if (n == 0 || total == 0) return GS_OK;
  GS_REQUIRE(bounds && order && offsets && tile_keys && gaussian_ids && aligned16(bounds),
             GS_ERR_INVALID_ARGUMENT, "null or misaligned pointer");
  emit_kernel<false><<<emit_blocks(total), kBlock, 0, as_stream(stream)>>>(
      reinterpret_cast<const int4*>(bounds), order, nullptr, 0, offsets, n, total, tiles_w,
      tile_keys, gaussian_ids);
  return check_launch("emit_tiles");
}

GS_API int gs_sort_tiles(uint32_t* tile_keys, int32_t* gaussian_ids, int64_t total,
                         int32_t num_tiles, int32_t* sorted_ids, int64_t* ranges, void* workspace,
                         size_t workspace_bytes, void* stream) {
  clear_error();
  GS_REQUIRE(total >= 0 && num_tiles > 0 && ranges, GS_ERR_INVALID_ARGUMENT,
             "invalid sort arguments");
  hipStream_t s = as_stream(stream);
  uint32_t* sorted_keys = tile_keys;
  if (total > 0) {
    GS_REQUIRE(tile_keys && gaussian_ids && sorted_ids, GS_ERR_INVALID_ARGUMENT, "null pointer");
    GS_REQUIRE(workspace_bytes >= sort_ws_bytes<uint32_t>(total), GS_ERR_WORKSPACE,
               "sort workspace too small");
    GS_TRY(radix_sort<uint32_t>(tile_keys, reinterpret_cast<const uint32_t*>(gaussian_ids), total,
                                bits_for(num_tiles), reinterpret_cast<uint32_t*>(sorted_ids),
                                &sorted_keys, workspace, workspace_bytes, s));
  }
  ranges_kernel<uint32_t, 0><<<unsigned(ceil_div(num_tiles, 256)), 256, 0, s>>>(
      sorted_keys, total, num_tiles, ranges);
  return check_launch("sort_tiles");
}

}  // extern "C"
