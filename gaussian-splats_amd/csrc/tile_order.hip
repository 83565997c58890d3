// Dispatch plan of the compositing tiles (DispatchPlan in common.h).
//
// The compositing kernels run one wave per work item, four items per
// workgroup, and map workgroups onto XCDs so that each XCD composites one
// region of the plan (xcd_swizzle).  A region is every eighth chunk of
// consecutive tiles (region_chunk): neighbouring tiles share Gaussians, which
// then stay in that XCD's L2, and a dense band of the image is spread over
// all eight XCDs (config 4, 4M Gaussians at 1600 x 1600, concentrates its
// work in the middle rows: with contiguous regions four XCDs idled while the
// other four walked it, 0.67 / 0.64 ms forward / backward; dealt, 0.61 /
// 0.47 ms).  Two things stretch a launch beyond its
// average wave: workgroups dispatched last (when not every wave fits on the
// GPU at once) that hold long tiles, and single tiles whose walk alone is
// longer than the rest of the launch (long lists in dense regions).  The plan
// keeps each XCD's region but sorts its tiles by decreasing expected work (to
// eight significant bits), so the long tiles start first and the short ones
// fill the tail (longest-processing-time-first list scheduling).  A backward
// plan also splits the region's heaviest tiles into kSegments items, each
// walking one segment of the tile's entries (composite_bwd.hip), so a tile
// whose walk is far longer than the rest no longer sets the launch's length;
// with few tiles every tile is split into the quarters of its pixel bands.
// Ties keep ascending tile index, so the plan is deterministic.
//
// Work estimates: the list length of the tile (forward), or the largest
// contributor count of its pixels (the entries the backward walks).
#include <algorithm>
#include <mutex>

#include "common.h"

namespace gs {
namespace {

constexpr int kOrderThreads = 1024;
constexpr int kOrderMax = 8192;  // tiles per region ordered by one workgroup

// key[t] = expected work of tile t, capped at 2^16 - 1, and crossings[t] =
// the forward checkpoints a backward walk of the tile crosses (with both
// n_contributors and ranges; else 0).  One wave per tile.
__global__ __launch_bounds__(256) void tile_key_kernel(const int64_t* __restrict__ ranges,
                                                       const int32_t* __restrict__ ncon,
                                                       int tiles_w, int num_tiles, int tile,
                                                       int width, int height, int view_tw,
                                                       int view_th, int cols, int views,
                                                       uint32_t* __restrict__ key,
                                                       uint32_t* __restrict__ crossings) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= num_tiles) return;
  int64_t work;
  if (ncon) {
    // Mosaic tile -> view and pixel origin inside it (see gs_view).
    const int tx = t % tiles_w, ty = t / tiles_w;
    const int vx = tx / view_tw, vy = ty / view_th;
    const int view = vy * cols + vx;
    const int ox = (tx - vx * view_tw) * tile, oy = (ty - vy * view_th) * tile;
    const int32_t* vn = ncon + int64_t(view < views ? view : 0) * width * height;
    int m = 0;
    for (int q = lane; view < views && q < tile * tile; q += 64) {
      const int px = ox + q % tile, py = oy + q / tile;
      if (px < width && py < height) m = max(m, vn[int64_t(py) * width + px]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = max(m, __shfl_xor(m, o, 64));
    work = m;
  } else {
    work = ranges[2 * t + 1] - ranges[2 * t];
  }
  if (lane == 0) {
    key[t] = uint32_t(min(max(work, int64_t(0)), int64_t(0xFFFF)));
    crossings[t] = ncon && ranges ? uint32_t(checkpoint_count(ranges[2 * t], int(work),
                                                              ranges[2 * t + 1] - ranges[2 * t]))
                                  : 0u;
  }
}

// Exclusive prefix sum over the 1024 threads' values (16 waves), in LDS
// scratch of 16 words; `total` receives the sum.  All threads take part.
__device__ __forceinline__ uint32_t block_exclusive(uint32_t v, uint32_t* scratch,
                                                    uint32_t& total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  uint32_t incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t u = uint32_t(__shfl_up(int(incl), o, 64));
    if (lane >= o) incl += u;
  }
  __syncthreads();  // scratch free (an earlier call may still read it)
  if (lane == 63) scratch[wid] = incl;
  __syncthreads();
  uint32_t before = 0, all = 0;
  for (int w = 0; w < 16; ++w) {
    const uint32_t c = scratch[w];
    before += w < wid ? c : 0u;
    all += c;
  }
  total = all;
  return before + incl - v;
}

// Region r of the order (the slots xcd_swizzle gives XCD r): chunks r, r + 8,
// r + 16, ... of region_chunk(num_tiles) tiles.  Its number of tiles, and its
// tile e.
__device__ __forceinline__ int region_size(int r, int num_tiles) {
  const int k = region_chunk(num_tiles);
  const int chunks = (num_tiles + k - 1) / k;
  const int mine = chunks > r ? (chunks - r + 7) / 8 : 0;
  if (mine == 0) return 0;
  const int last = r + 8 * (mine - 1);
  return (mine - 1) * k + min(k, num_tiles - last * k);
}
__device__ __forceinline__ int region_tile(int r, int e, int k) {
  return ((e / k) * 8 + r) * k + e % k;
}

// One workgroup per region: a stable counting sort of the region's tiles by
// the eight most significant bits of the key (relative to the region's largest
// key), largest first, then the region's items in that order, each tile as
// 1 + extra items: extra = 3 (its four quarters) when the plan splits every
// tile, else its checkpoint crossings (1 + crossings segments) while the
// region's spare slots last, heaviest tiles first, else 0 (whole).  Sixteen
// waves take contiguous index segments; a wave ranks its tiles per bucket
// with ballots (eight, one per digit bit), so ties keep index order.  Unused
// slots of the region get -1.
__global__ __launch_bounds__(kOrderThreads) void tile_plan_kernel(
    const uint32_t* __restrict__ key, const uint32_t* __restrict__ crossings, int num_tiles,
    int segments, int split_all, int region_slots, int32_t* __restrict__ items) {
  constexpr int kWaves = kOrderThreads / 64;
  constexpr int kPerLane = kOrderMax / kOrderThreads;  // tiles per lane at most
  __shared__ uint32_t cnt[kWaves][256];
  __shared__ uint32_t start[256];
  __shared__ uint32_t smax, scratch[kWaves];
  __shared__ int32_t sorted_tile[kOrderMax];
  __shared__ uint8_t sorted_extra[kOrderMax];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int r = blockIdx.x;
  const int n = region_size(r, num_tiles);
  const int rk = region_chunk(num_tiles);
  int32_t* out = items + int64_t(blockIdx.x) * region_slots;
  if (n > kOrderMax) {  // too large to sort here: index order, no segments
    const int per = split_all ? 4 : 1;
    for (int i = threadIdx.x; i < n * per; i += kOrderThreads)
      out[i] = split_all ? (region_tile(r, i / 4, rk) << 7 | 0x20 | (i & 3))
                         : region_tile(r, i, rk) << 7;
    for (int i = n * per + threadIdx.x; i < region_slots; i += kOrderThreads) out[i] = -1;
    return;
  }
  if (threadIdx.x == 0) smax = 0;
  for (int i = threadIdx.x; i < kWaves * 256; i += kOrderThreads) (&cnt[0][0])[i] = 0;
  __syncthreads();
  const int seg = (n + kWaves - 1) / kWaves;  // <= kPerLane * 64
  const int s0 = wid * seg, s1 = min(s0 + seg, n);
  uint32_t k[kPerLane];
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const int e = s0 + i * 64 + lane;
    k[i] = e < s1 ? key[region_tile(r, e, rk)] : 0u;
    m = max(m, k[i]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = max(m, uint32_t(__shfl_xor(int(m), o, 64)));
  if (lane == 0) atomicMax(&smax, m);
  __syncthreads();
  const int shift = max(0, 24 - __clz(int(smax | 1u)));  // smax >> shift < 256
  uint32_t dig[kPerLane], rank[kPerLane];
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    dig[i] = 255u - (k[i] >> shift);
    rank[i] = 0;
  }
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    // Rounds past the wave's segment hold no tile (a region of n tiles fills
    // ceil(n / 1024) of the eight): skipped, wave-uniformly.
    if (s0 + i * 64 >= s1) break;
    const int e = s0 + i * 64 + lane;
    const bool valid = e < s1;
    uint32_t plo = uint32_t(__ballot(valid)), phi = uint32_t(__ballot(valid) >> 32);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const uint32_t mb = uint32_t(int32_t(dig[i] << (31 - bit)) >> 31);
      const uint64_t ones = __ballot(mb != 0u);
      plo &= ~(uint32_t(ones) ^ mb);
      phi &= ~(uint32_t(ones >> 32) ^ mb);
    }
    const uint32_t before = __builtin_amdgcn_mbcnt_hi(phi, __builtin_amdgcn_mbcnt_lo(plo, 0u));
    const uint32_t total = uint32_t(__popc(plo) + __popc(phi));
    uint32_t c = 0;
    if (valid) {
      c = cnt[wid][dig[i]];
      cnt[wid][dig[i]] = c + total;
    }
    rank[i] = c + before;
  }
  __syncthreads();
  // Bucket starts: digit-major over the waves, in one wave.
  if (wid == 0) {
    uint32_t carry = 0;
    for (int d0 = 0; d0 < 256; d0 += 64) {
      const int d = d0 + lane;
      uint32_t tot = 0;
      for (int w = 0; w < kWaves; ++w) {
        const uint32_t c = cnt[w][d];
        cnt[w][d] = tot;  // wave offset within the bucket
        tot += c;
      }
      uint32_t incl = tot;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = uint32_t(__shfl_up(int(incl), o, 64));
        if (lane >= o) incl += v;
      }
      start[d] = carry + incl - tot;
      carry += uint32_t(__shfl(int(incl), 63, 64));
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const int e = s0 + i * 64 + lane;
    if (e < s1) {
      const int p = int(start[dig[i]] + cnt[wid][dig[i]] + rank[i]);  // sorted position
      const int t = region_tile(r, e, rk);
      sorted_tile[p] = t;
      sorted_extra[p] = uint8_t(split_all ? 3u : segments ? min(crossings[t], 63u) : 0u);
    }
  }
  __syncthreads();
  // Thread i takes sorted positions [kPerLane i, kPerLane i + kPerLane).
  const int p0 = int(threadIdx.x) * kPerLane;
  uint32_t ex[kPerLane], sum = 0;
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    ex[i] = p0 + i < n ? uint32_t(sorted_extra[p0 + i]) : 0u;
    sum += ex[i];
  }
  // Spare slots go to the tiles in sorted order while they fit whole.
  uint32_t all;
  uint32_t before = block_exclusive(sum, scratch, all);
  const uint32_t spare = uint32_t(region_slots - n);
  sum = 0;
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    if (before + ex[i] > spare) ex[i] = 0;  // does not fit: whole
    before += ex[i];
    sum += ex[i];
  }
  // Item offsets of the final counts (1 + extra per tile).
  uint32_t used;
  uint32_t off = block_exclusive(sum, scratch, used) + uint32_t(p0);
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    if (p0 + i < n) {
      const int t = sorted_tile[p0 + i];
      if (ex[i] == 0) {
        out[off] = t << 7;
      } else {
        const int code = split_all ? 0x20 : 0x40;
        for (uint32_t j = 0; j <= ex[i]; ++j) out[off + j] = t << 7 | code | int(j);
      }
      off += 1 + ex[i];
    }
  }
  for (int i = n + int(used) + threadIdx.x; i < region_slots; i += kOrderThreads) out[i] = -1;
}

}  // namespace
}  // namespace gs

using namespace gs;

// Scratch memory of gs_tile_order_noalloc: the per-tile work keys and
// checkpoint crossings.  One copy per GPU (each at its own device address),
// held until the process ends.
constexpr int kNoAllocMaxTiles = GS_TILE_ORDER_NOALLOC_MAX_TILES;  // 2 MiB of keys
static __device__ __align__(256) uint32_t scratch[2 * kNoAllocMaxTiles];

namespace {

constexpr int kScratchDevices = 64;
uint32_t* g_scratch_addr[kScratchDevices] = {};
std::mutex g_scratch_mutex;

// Device address of `scratch` on the stream's GPU.  The host-side name of the
// array is not a device address; it is looked up once per device, with that
// device current, and only the looked-up address is handed to kernels.
int scratch_keys(hipStream_t stream, uint32_t** keys) {
  int device = 0;
  GS_TRY(stream_device(stream, &device));
  GS_REQUIRE(device < kScratchDevices, GS_ERR_HIP, "device %d out of range", device);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_addr[device]) {
    int current = 0;
    GS_REQUIRE(hipGetDevice(&current) == hipSuccess, GS_ERR_HIP, "hipGetDevice failed");
    const bool switch_device = current != device;
    if (switch_device) GS_REQUIRE(hipSetDevice(device) == hipSuccess, GS_ERR_HIP, "hipSetDevice");
    void* addr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (switch_device) (void)hipSetDevice(current);
    GS_REQUIRE(e == hipSuccess && addr, GS_ERR_HIP, "tile order scratch lookup failed: %s",
               hipGetErrorString(e));
    g_scratch_addr[device] = static_cast<uint32_t*>(addr);
  }
  *keys = g_scratch_addr[device];
  return GS_OK;
}

// Both kernels on `s`: keys for every tile, then the per-region plans.
// Every key the plan kernel reads is written by the key kernel of the same
// call, or, with keys_ready, by the forward compositing that produced
// n_contributors (gs_composite's tile_keys: whole-tile walks write every
// tile's key), so `key` needs no clearing.
int tile_order_launch(const int64_t* ranges, const int32_t* n_contributors, const gs_view& view,
                      const Mosaic& m, int32_t* items, uint32_t* key, bool keys_ready,
                      hipStream_t s) {
  const int num_tiles = m.num_tiles();
  GS_REQUIRE(num_tiles < (1 << 24), GS_ERR_OVERFLOW, "too many tiles (%d)", num_tiles);
  const DispatchPlan plan =
      dispatch_plan(num_tiles, view.tile_size, view.active_tiles, n_contributors != nullptr);
  uint32_t* crossings = key + num_tiles;
  // The forward writes keys only when it walked whole tiles.
  const bool forward_keys = keys_ready && n_contributors &&
                            !dispatch_plan(num_tiles, view.tile_size, view.active_tiles, false)
                                 .split_all;
  if (!forward_keys) {
    tile_key_kernel<<<unsigned(ceil_div(num_tiles, 4)), 256, 0, s>>>(
        ranges, n_contributors, m.tiles_w(), num_tiles, view.tile_size, view.image_width,
        view.image_height, m.tw, m.th, m.cols, m.views, key, crossings);
    GS_TRY(check_launch("tile_order keys"));
  }
  tile_plan_kernel<<<8, kOrderThreads, 0, s>>>(key, crossings, num_tiles,
                                                plan.segments ? 1 : 0, plan.split_all ? 1 : 0,
                                                plan.items() / 8, items);
  return check_launch("tile_order plan");
}

}  // namespace

extern "C" {

GS_API size_t gs_tile_order_workspace_bytes(int32_t num_tiles) {
  return num_tiles > 0 ? align_up(size_t(num_tiles) * 2 * sizeof(uint32_t)) : 0;
}

GS_API int64_t gs_tile_order_items(gs_view view, int32_t by_contributors) {
  clear_error();
  if (check_view(view, true) != GS_OK) return -1;
  const Mosaic m = mosaic_of(view);
  return dispatch_plan(m.num_tiles(), view.tile_size, view.active_tiles, by_contributors != 0)
      .items();
}

GS_API int gs_tile_order(const int64_t* ranges, const int32_t* n_contributors, gs_view view,
                         int32_t* order, void* workspace, size_t workspace_bytes,
                         int32_t keys_ready, void* stream) {
  clear_error();
  GS_TRY(check_view(view, true));
  const Mosaic m = mosaic_of(view);
  const int num_tiles = m.num_tiles();
  GS_REQUIRE(order && (ranges || n_contributors), GS_ERR_INVALID_ARGUMENT,
             "null pointer argument");
  GS_REQUIRE(workspace && workspace_bytes >= gs_tile_order_workspace_bytes(num_tiles),
             GS_ERR_WORKSPACE, "workspace too small (%zu bytes, need %zu)", workspace_bytes,
             gs_tile_order_workspace_bytes(num_tiles));
  return tile_order_launch(ranges, n_contributors, view, m, order,
                           static_cast<uint32_t*>(workspace), keys_ready != 0,
                           as_stream(stream));
}

GS_API int gs_tile_order_noalloc(const int64_t* ranges, const int32_t* n_contributors,
                                 gs_view view, int32_t* order, void* stream) {
  clear_error();
  GS_TRY(check_view(view, true));
  const Mosaic m = mosaic_of(view);
  const int num_tiles = m.num_tiles();
  GS_REQUIRE(order && (ranges || n_contributors), GS_ERR_INVALID_ARGUMENT,
             "null pointer argument");
  GS_REQUIRE(num_tiles <= kNoAllocMaxTiles, GS_ERR_WORKSPACE,
             "gs_tile_order_noalloc: %d tiles exceed its static scratch of %d tiles "
             "(use gs_tile_order with a workspace)",
             num_tiles, kNoAllocMaxTiles);
  const hipStream_t s = as_stream(stream);
  uint32_t* keys = nullptr;
  GS_TRY(scratch_keys(s, &keys));
  return tile_order_launch(ranges, n_contributors, view, m, order, keys, false, s);
}

}  // extern "C"
