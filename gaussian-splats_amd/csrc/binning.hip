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
// Sorts and scans are the single-pass kernels of onesweep.h.
#include "block_scan.h"
#include "common.h"
#include "onesweep.h"
#include "radix.h"

namespace gs {
namespace {



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

GS_API size_t gs_scan_workspace_bytes(int64_t n) {
  return carve(nullptr, 0, 4, -1, n < 0 ? 0 : n).bytes;
}

GS_API int gs_scan_counts(const int32_t* counts, int64_t n, int64_t* offsets, void* workspace,
                          size_t workspace_bytes, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0 && offsets && (n == 0 || counts), GS_ERR_INVALID_ARGUMENT,
             "invalid scan arguments");
  hipStream_t s = as_stream(stream);
  if (n == 0) {
    fill_kernel<int64_t><<<1, 64, 0, s>>>(offsets, 1, 0);
    return check_launch("scan_counts");
  }
  Scratch ws = carve(workspace, 0, 4, -1, n);
  GS_REQUIRE(workspace && workspace_bytes >= ws.bytes, GS_ERR_WORKSPACE, "scan workspace too small");
  GS_TRY(device_flags(s, &ws.flags));
  clear(ws, s);
  launch_scan<int64_t>(sweep::GatherLoad<int32_t, int64_t>{counts, nullptr}, n, offsets, true,
                       aligned_16(counts), ws, s);
  return check_launch("scan_counts");
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
  if (total < 0) total = 0;
  // Enough for either key format: 64-bit reference keys over 32 + tile bits.
  return carve(nullptr, total, 8, 32 + bits_for(std::max(1, num_tiles)), 0).bytes;
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
    const int end_bit = 32 + bits_for(num_tiles);
    Scratch ws = carve(workspace, total, 8, end_bit, 0);
    GS_REQUIRE(workspace && workspace_bytes >= ws.bytes, GS_ERR_WORKSPACE,
               "sort workspace too small (%zu < %zu)", workspace_bytes, ws.bytes);
    GS_TRY(device_flags(s, &ws.flags));
    clear(ws, s);
    GS_TRY(radix_sort<uint64_t>(reinterpret_cast<uint64_t*>(keys),
                                reinterpret_cast<const uint32_t*>(gaussian_ids), total, end_bit,
                                reinterpret_cast<uint32_t*>(sorted_ids), &sorted_keys, ws, s));
  }
  ranges_kernel<uint64_t, 32><<<unsigned(ceil_div(num_tiles, 256)), 256, 0, s>>>(
      sorted_keys, total, num_tiles, ranges);
  return check_launch("sort_intersections");
}

GS_API size_t gs_bin_workspace_bytes(int64_t n) {
  if (n < 0) n = 0;
  return carve(nullptr, n, 4, 32, n).bytes;
}

GS_API int gs_bin_gaussians(uint32_t* depth_keys, const int32_t* counts, int64_t n,
                            int32_t* order, int64_t* offsets, void* workspace,
                            size_t workspace_bytes, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0 && offsets, GS_ERR_INVALID_ARGUMENT, "invalid binning arguments");
  hipStream_t s = as_stream(stream);
  if (n == 0) {
    fill_kernel<int64_t><<<1, 64, 0, s>>>(offsets, 1, 0);
    return check_launch("bin_gaussians");
  }
  GS_REQUIRE(depth_keys && counts && order, GS_ERR_INVALID_ARGUMENT, "null pointer");
  Scratch ws = carve(workspace, n, 4, 32, n);
  GS_REQUIRE(workspace && workspace_bytes >= ws.bytes, GS_ERR_WORKSPACE,
             "binning workspace too small");
  GS_TRY(device_flags(s, &ws.flags));
  clear(ws, s);
  // depth_keys is used as a ping-pong buffer by the sort and is consumed.
  uint32_t* sorted_keys = nullptr;
  GS_TRY((radix_sort<uint32_t, true>)(depth_keys, nullptr, n, 32, reinterpret_cast<uint32_t*>(order),
                              &sorted_keys, ws, s));
  launch_scan<int64_t>(sweep::GatherLoad<int32_t, int64_t>{counts, order}, n, offsets, true,
                       aligned_16(order), ws, s);
  return check_launch("bin_gaussians");
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
    const int end_bit = bits_for(num_tiles);
    Scratch ws = carve(workspace, total, 4, end_bit, 0);
    GS_REQUIRE(workspace && workspace_bytes >= ws.bytes, GS_ERR_WORKSPACE,
               "sort workspace too small");
    GS_TRY(device_flags(s, &ws.flags));
    clear(ws, s);
    GS_TRY(radix_sort<uint32_t>(tile_keys, reinterpret_cast<const uint32_t*>(gaussian_ids), total,
                                end_bit, reinterpret_cast<uint32_t*>(sorted_ids), &sorted_keys,
                                ws, s));
  }
  ranges_kernel<uint32_t, 0><<<unsigned(ceil_div(num_tiles, 256)), 256, 0, s>>>(
      sorted_keys, total, num_tiles, ranges);
  return check_launch("sort_tiles");
}

}  // extern "C"
