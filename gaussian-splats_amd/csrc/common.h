// Shared host/device helpers for the gfx950 rasterizer kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>

#include "gs_raster.h"

namespace gs {

// Per-thread error message behind gs_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Checks the launch that was just enqueued; converts a HIP error into a status.
int check_launch(const char* what);

// Work forked from the caller's stream onto the library's side stream of the
// same device (created once, default priority, non-blocking) and joined back
// with an event, so two independent stages overlap.  The side stream is held
// exclusively from fork to join.
struct SideFork {
  hipStream_t main = nullptr;
  hipStream_t side = nullptr;
  hipEvent_t mark = nullptr;
  hipEvent_t join = nullptr;
  std::unique_lock<std::mutex> lock;
};
int fork_side_stream(hipStream_t main, SideFork& f);
// One intermediate dependency: record_side_mark marks the side stream's work
// enqueued so far; work enqueued on the caller's stream after
// wait_side_mark waits for it.
int record_side_mark(SideFork& f);
int wait_side_mark(SideFork& f);
// Joins the side stream back into the caller's; with host_wait the host also
// waits for the side stream's work (not the caller's) before returning.
int join_side_stream(SideFork& f, bool host_wait = false);

// Device of a stream (the current device for the null stream).
int stream_device(hipStream_t stream, int* device);

// Address of the stream's device's sticky check-failure word (see
// gs_device_errors): kernels OR kDeviceFlag* bits into it.
int device_flags(hipStream_t stream, uint32_t** flags);
constexpr uint32_t kDeviceFlagSpinLimit = GS_DEVICE_SPIN_LIMIT;
constexpr uint32_t kDeviceFlagWindow = GS_DEVICE_WINDOW_OVERFLOW;
constexpr uint32_t kDeviceFlagSizes = GS_DEVICE_SIZE_MISMATCH;

#define GS_REQUIRE(cond, code, ...)      \
  do {                                   \
    if (!(cond)) {                       \
      ::gs::set_error(__VA_ARGS__);      \
      return (code);                     \
    }                                    \
  } while (0)

#define GS_TRY(expr)                     \
  do {                                   \
    int gs_status_ = (expr);             \
    if (gs_status_ != GS_OK) return gs_status_; \
  } while (0)

constexpr int kWave = 64;

// Waves (tiles) per workgroup of the compositing kernels; the tile dispatch
// order of tile_order.hip partitions the tiles the same way.
constexpr int kCompositeWaves = 4;

// Images with fewer tiles with work than this are composited with the tile's
// bands split over kCompositeWaves waves (tiles of 16 and 32 pixels): with one
// wave per tile they would leave most SIMDs idle and wait on their longest
// tiles.  `active` counts the tiles with a non-empty list (0: unknown, all).
constexpr int kCompositeSplitTiles = 4096;
inline bool composite_split(int num_tiles, int active) {
  return (active > 0 && active < num_tiles ? active : num_tiles) < kCompositeSplitTiles;
}

// Dispatch plan of the compositing kernels (gs_tile_order).  Each of the 8
// XCD regions of tiles (a contiguous range of tile indices) owns the same
// number of item slots; an item is one wave's work:
//   tile << 3                      the whole tile, or
//   tile << 3 | 4 | band           a quarter of its pixel bands (tiles of 16
//                                  and 32 pixels); the four quarters of a tile
//                                  fill the four slots of one workgroup,
// and -1 marks an unused slot.  With few tiles (composite_split) every tile is
// split.  Splitting only a region's heaviest tiles (kSplitHeavy: above
// kHeavyNum / kHeavyDen of the region's mean, at most one in kHeavyShare) is
// implemented but off: as four independent waves, the quarters of a heavy
// tile add their gradients with four times the atomics on the Gaussians they
// share (config 4's backward went from 1.77 to 3.0 ms), and the forward's
// list-length estimate misses the tiles whose walks are longest.
constexpr bool kSplitHeavy = false;
constexpr int kHeavyShare = 8;
constexpr int kHeavyNum = 3, kHeavyDen = 2;
struct DispatchPlan {
  bool heavy = false;      // a region's heaviest tiles split into quarters
  bool split_all = false;  // every tile split into quarters
  int region_blocks = 1;   // workgroups (of kCompositeWaves items) per region
  int items() const { return 8 * kCompositeWaves * region_blocks; }
};
inline DispatchPlan dispatch_plan(int num_tiles, int tile_size, int active) {
  DispatchPlan p;
  const bool bands = tile_size >= 16;
  p.split_all = bands && composite_split(num_tiles, active);
  p.heavy = bands && kSplitHeavy && !p.split_all;
  // Tiles of the largest region (tile_order.hip's region split).
  const int nb = (num_tiles + kCompositeWaves - 1) / kCompositeWaves;
  const int t_max = (nb + 7) / 8 * kCompositeWaves;
  const int cap = p.split_all ? 4 * t_max
                  : p.heavy   ? t_max + 3 * ((t_max + kHeavyShare - 1) / kHeavyShare)
                              : t_max;
  p.region_blocks = cap > kCompositeWaves ? (cap + kCompositeWaves - 1) / kCompositeWaves : 1;
  return p;
}

// The work item of compositing slot `slot` (kCompositeWaves per workgroup):
// from the plan's items, or, without a plan, tile `slot` whole (or its
// quarter slot % 4 of tile slot / 4 when every tile is split).  False: no
// work (an unused slot, or a tile index out of range).
__device__ __forceinline__ bool composite_item(const int32_t* items, int num_items,
                                               int num_tiles, bool split_all, int slot,
                                               int& tile, int& band, bool& quarter) {
  if (items) {
    if (slot >= num_items) return false;
    const int it = items[slot];
    if (it < 0) return false;
    tile = it >> 3;
    quarter = (it & 4) != 0;
    band = it & 3;
  } else if (split_all) {
    tile = slot >> 2;
    band = slot & 3;
    quarter = true;
  } else {
    tile = slot;
    band = 0;
    quarter = false;
  }
  return tile < num_tiles;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline size_t align_up(size_t x, size_t a = 256) { return (x + a - 1) / a * a; }

// Number of tiles along each axis (partial tiles at the right/bottom edge).
inline int tiles_along(int pixels, int tile) { return (pixels + tile - 1) / tile; }

inline bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

// Validates the geometry part of a gs_view.
int check_view(const gs_view& v, bool need_tiles);

// Tile layout of a (possibly multi-view) gs_view: each view has tw x th
// tiles; the mosaic is cols x rows views.
struct Mosaic {
  int views, cols, rows, tw, th;
  int tiles_w() const { return cols * tw; }
  int tiles_h() const { return rows * th; }
  int num_tiles() const { return tiles_w() * tiles_h(); }
};
inline Mosaic mosaic_of(const gs_view& v) {
  Mosaic m;
  m.views = v.views > 1 ? v.views : 1;
  m.cols = v.mosaic_cols > 1 ? v.mosaic_cols : 1;
  if (m.cols > m.views) m.cols = m.views;
  m.rows = (m.views + m.cols - 1) / m.cols;
  m.tw = tiles_along(v.image_width, v.tile_size);
  m.th = tiles_along(v.image_height, v.tile_size);
  return m;
}

// Maps a linear workgroup index onto a work index so that consecutive work
// items land on the same XCD.  Workgroups are dispatched round-robin over the
// 8 XCDs (b % 8 selects the XCD); XCD x receives q + (x < r) workgroups
// (q = nb / 8, r = nb % 8), which are given the contiguous work range starting
// at x * q + min(x, r).  The map is a bijection of [0, nb).
__device__ __forceinline__ int xcd_swizzle(int b, int nb) {
  const int q = nb >> 3, r = nb & 7;
  const int x = b & 7;
  return x * q + min(x, r) + (b >> 3);
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int lane = __lane_id();
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

}  // namespace gs

// Packed per-Gaussian compositing record (48 bytes, three dwordx4 loads).
struct __attribute__((aligned(16))) GsRecord {
  float u, v, opacity, depth;
  float inv00, inv01, inv11, cut;  // cut: largest quadratic form with alpha >= 1/255
  float r, g, b, pad;
};
static_assert(sizeof(GsRecord) == 48, "record layout");
