// Shared host/device helpers for the gfx950 rasterizer kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
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

// Timing events armed for the next launch_timed() call of the calling thread
// (gs_arm_launch_events).  Taking them disarms them, so one armed pair times
// exactly one kernel.
struct LaunchEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
LaunchEvents take_launch_events();

template <typename T>
struct NoDeduce {
  using type = T;
};

// Launches `kernel`; with armed events the launch carries them
// (hipExtLaunchKernel), so they take the kernel's own start and end
// timestamps and no marker packet is queued before or after it.
template <typename... Params>
void launch_timed(void (*kernel)(Params...), dim3 grid, dim3 block, uint32_t lds, hipStream_t s,
                  typename NoDeduce<Params>::type... args) {
  const LaunchEvents ev = take_launch_events();
  if (!ev.start && !ev.stop) {
    kernel<<<grid, block, lds, s>>>(args...);
    return;
  }
  void* argv[] = {static_cast<void*>(&args)...};
  // A failure is left in hipGetLastError for the caller's check_launch.
  (void)hipExtLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, argv, lds, s,
                           ev.start, ev.stop, 0);
}

// Work forked from the caller's stream onto the library's side stream of the
// same device and calling thread (created on the thread's first fork on that
// device, default priority, non-blocking) and joined back with an event, so
// two independent stages overlap.  Each thread has its own side stream and
// events: calls from several threads on one GPU neither share nor wait for
// them.
struct SideFork {
  hipStream_t main = nullptr;
  hipStream_t side = nullptr;
  hipEvent_t join = nullptr;
};
int fork_side_stream(hipStream_t main, SideFork& f);
// Joins the side stream back into the caller's: the caller's stream waits
// for the side stream's work, or, with host_wait, the host does (not for the
// caller's stream) before returning, after which anything enqueued on the
// caller's stream follows the side stream's work.
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

// Loads of data a kernel reads exactly once (the projection's parameters,
// coefficient blocks and gradient inputs, the loss's image and target): the
// nontemporal hint streams the lines through the caches instead of retaining
// them.  On 1M Gaussians of SH degree 3 the projection went from 72 to 61 us
// with it, its backward from 98 to 89 us, the L1 loss from 11.8 to 10.3 us.
// (Measured no faster on the sort's key reads and the bucketing passes'
// list reads, which keep their plain loads.)
typedef float float4_ext __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float load_nt(const float* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ int32_t load_nt(const int32_t* p) {
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ uint32_t load_nt(const uint32_t* p) {
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ uint64_t load_nt(const uint64_t* p) {
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ float4 load_nt(const float4* p) {
  const float4_ext v = __builtin_nontemporal_load(reinterpret_cast<const float4_ext*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
// Stores of results no kernel of the step reads again (the parameter
// gradients): the nontemporal hint keeps them from displacing cached lines
// (config 3: projection backward 91 -> 90 us, and the next step's projection
// 60 -> 57 us; the optimiser step that reads them took as long).
__device__ __forceinline__ void store_nt(float v, float* p) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void store_nt(const float4& v, float4* p) {
  __builtin_nontemporal_store(float4_ext{v.x, v.y, v.z, v.w}, reinterpret_cast<float4_ext*>(p));
}

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

// Checkpoints of the forward walk (composite_fwd.hip) that let the backward
// walk a long list in segments.  Whenever a whole-tile wave of a list longer
// than kCheckpointMinList starts a batch of 64 entries that holds a list
// position P = j * kCheckpointEntries of the intersection array (P at least
// 64 past the tile's first entry), it records
// per pixel the transmittance and the colour composited since its previous
// checkpoint, and at the end of the walk turns the colours into the colour
// composited after each checkpoint (a suffix sum, so the backward starts a
// segment with g.S = g . C_after / T and no difference of rounded sums).  At
// most kMaxCheckpoints per tile; records come from a pool (a device counter
// and kCheckpointPoolBytes of records), slot j of the table holding the
// record of position j * kCheckpointEntries (-1: the pool was full).
constexpr int kCheckpointEntries = 1024;
constexpr int kMaxCheckpoints = 63;
// Only tiles with longer lists record checkpoints: shorter walks are not
// worth the records and the extra items (measured on config 3, whose lists
// reach ~7000 entries: checkpoints on every tile cost 9 us of forward and
// 17 us of backward).
constexpr int kCheckpointMinList = 8192;
constexpr size_t kCheckpointPoolBytes = size_t(128) << 20;

// Pixels of a tile's checkpoint record (64 for tiles of fewer pixels).
inline int checkpoint_pixels(int tile_size) {
  return tile_size * tile_size >= 64 ? tile_size * tile_size : 64;
}

// Layout of the checkpoint workspace: a 256-byte header block (the pool
// counter, then the stamp), the table, the records.  The records fill what
// the caller's buffer holds beyond the header and table, up to one per table
// slot and kCheckpointPoolBytes: a smaller buffer holds fewer records, and the
// crossings beyond them are recorded as missing (-1).
struct CheckpointLayout {
  uint32_t* counter = nullptr;
  uint32_t* stamp = nullptr;  // kCheckpointStampWords words after the counter
  int32_t* table = nullptr;
  float4* records = nullptr;
  int64_t table_len = 0;
  int64_t capacity = 0;     // records
  size_t header_bytes = 0;  // header block + table: the least a buffer must hold
  size_t bytes = 0;         // header + records
};
// The stamp says which walk wrote the table: the forward writes it with its
// pool counter before the walk (or clears it when it records nothing into a
// buffer it is given), and the backward trusts the table only when the stamp
// matches its own view.  It cannot tell two walks of one geometry apart: the
// buffer must come from the forward over the same lists.
constexpr uint32_t kCheckpointMagic = 0x70636773u;  // "sgcp"
constexpr int kCheckpointStampWords = 4;  // magic, tile size, tiles, table length
inline CheckpointLayout checkpoint_layout(void* base, int tile_size, int64_t total,
                                          size_t available = ~size_t(0)) {
  CheckpointLayout c;
  const size_t record = size_t(checkpoint_pixels(tile_size)) * 16;
  // A crossing's position lies below the list end + 64 (its batch starts
  // inside the list): table slots up to (total + 63) / kCheckpointEntries.
  c.table_len = total / kCheckpointEntries + 2;
  char* p = static_cast<char*>(base);
  size_t off = 0;
  auto take = [&](size_t n) {
    char* r = p ? p + off : nullptr;
    off += (n + 255) / 256 * 256;
    return r;
  };
  c.counter = reinterpret_cast<uint32_t*>(take(4 * (1 + kCheckpointStampWords)));
  c.stamp = c.counter ? c.counter + 1 : nullptr;
  c.table = reinterpret_cast<int32_t*>(take(size_t(c.table_len) * 4));
  c.header_bytes = off;
  const int64_t most = c.table_len;  // one record per table slot at most
  const int64_t room = available > off ? int64_t((available - off) / record) : 0;
  c.capacity = std::min<int64_t>(std::min<int64_t>(most, int64_t(kCheckpointPoolBytes / record)),
                                 room);
  c.records = reinterpret_cast<float4*>(take(size_t(c.capacity) * record));
  c.bytes = off;
  return c;
}

// Dispatch plan of the compositing kernels (gs_tile_order).  Each of the 8
// XCD regions of tiles (a contiguous range of tile indices) owns the same
// number of item slots; an item is one wave's work, tile << 7 | code:
//   code 0            the whole tile;
//   code 0x20 | q     quarter q of its pixel bands (tiles of 16 and 32 pixels,
//                     when fewer than kCompositeSplitTiles tiles have work:
//                     every tile split, its quarters in one workgroup's slots);
//   code 0x40 | s     segment s of the entries a tile's pixels walk back
//                     (backward plans with the tile ranges): the walk is cut
//                     at the forward's checkpoints, the segments of a tile in
//                     consecutive slots;
// and -1 marks an unused slot.  A backward plan segments the tiles with
// checkpoints, heaviest first, while the region's spare slots last.
constexpr int kSegmentSpare = 4;  // spare slots per region, in units of its tiles
struct DispatchPlan {
  bool segments = false;   // tiles walked back in segments
  bool split_all = false;  // every tile split into quarters
  int region_blocks = 1;   // workgroups (of kCompositeWaves items) per region
  int items() const { return 8 * kCompositeWaves * region_blocks; }
};
// The plan deals the tiles to the 8 XCD regions in chunks of
// region_chunk(num_tiles) consecutive tiles (a multiple of kCompositeWaves,
// about eight chunks per region, at most 64 tiles), chunk c to region c % 8:
// a dense band of the image is spread over every XCD, while the tiles of a
// chunk (neighbours that share Gaussians) stay in one XCD's L2.
__host__ __device__ inline int region_chunk(int num_tiles) {
  const int k = (num_tiles + 63) / 64;
  return k < kCompositeWaves ? kCompositeWaves : k > 64 ? 64 : (k + kCompositeWaves - 1) & ~(kCompositeWaves - 1);
}
// Tiles of the largest region (region 0).
__host__ __device__ inline int region_max_tiles(int num_tiles) {
  const int k = region_chunk(num_tiles);
  const int chunks = (num_tiles + k - 1) / k;
  return (chunks + 7) / 8 * k;
}
inline DispatchPlan dispatch_plan(int num_tiles, int tile_size, int active, bool backward) {
  DispatchPlan p;
  p.split_all = tile_size >= 16 && composite_split(num_tiles, active);
  p.segments = backward && !p.split_all;
  const int t_max = region_max_tiles(num_tiles);
  const int cap = p.split_all ? 4 * t_max : p.segments ? (1 + kSegmentSpare) * t_max : t_max;
  p.region_blocks = cap > kCompositeWaves ? (cap + kCompositeWaves - 1) / kCompositeWaves : 1;
  return p;
}

// Kinds of compositing work item.
enum : int { kItemTile = 0, kItemQuarter = 1, kItemSegment = 2 };

// The work item of compositing slot `slot` (kCompositeWaves per workgroup):
// from the plan's items, or, without a plan, tile `slot` whole (or its
// quarter slot % 4 of tile slot / 4 when every tile is split).  False: no
// work (an unused slot, or a tile index out of range).  `index` is the
// quarter or segment.
__device__ __forceinline__ bool composite_item(const int32_t* items, int num_items,
                                               int num_tiles, bool split_all, int slot,
                                               int& tile, int& kind, int& index) {
  if (items) {
    if (slot >= num_items) return false;
    const int it = items[slot];
    if (it < 0) return false;
    tile = it >> 7;
    kind = (it & 0x40) ? kItemSegment : (it & 0x20) ? kItemQuarter : kItemTile;
    index = it & 0x1F;
    if (kind == kItemSegment) index = it & 0x3F;
  } else if (split_all) {
    tile = slot >> 2;
    kind = kItemQuarter;
    index = slot & 3;
  } else {
    tile = slot;
    kind = kItemTile;
    index = 0;
  }
  return tile < num_tiles;
}

// The checkpoint crossings of a tile whose list starts at `start` and whose
// pixels walk max_n entries: crossing j >= 1 is list position
// P_j = first + (j - 1) kCheckpointEntries (first: the first multiple of
// kCheckpointEntries at least 64 past start), recorded at the start of the
// batch holding it, B_j = 64 floor((P_j - start) / 64) entries into the walk,
// for the B_j < max_n (at most kMaxCheckpoints; none for lists of at most
// kCheckpointMinList entries).
__host__ __device__ inline int64_t checkpoint_first(int64_t start) {
  return (start + 64 + kCheckpointEntries - 1) / kCheckpointEntries * kCheckpointEntries;
}
__host__ __device__ inline int checkpoint_batch(int64_t start, int j) {  // B_j, j >= 1
  return int((checkpoint_first(start) + int64_t(j - 1) * kCheckpointEntries - start) / 64 * 64);
}
__host__ __device__ inline int checkpoint_count(int64_t start, int max_n, int64_t list_len) {
  const int64_t first = checkpoint_first(start) - start;  // >= 64
  if (max_n <= 64 || list_len <= kCheckpointMinList) return 0;
  // B_j < max_n  <=>  64 floor((first + (j-1) L) / 64) < max_n
  const int64_t limit = (int64_t(max_n) + 63) / 64 * 64;  // B_j < max_n <=> first + (j-1)L < limit
  if (first >= limit) return 0;
  const int64_t m = (limit - 1 - first) / kCheckpointEntries + 1;
  return int(m < kMaxCheckpoints ? m : kMaxCheckpoints);
}

// Hit masks (no counterpart in the reference): for every batch of 64 entries
// of a tile's list that the forward walks, one 64-bit mask per 64-pixel band
// of the tile (tile_bands), bit j set when entry j of the batch took a
// nonzero alpha at a pixel of the band while the pixel was active.  The masks
// of batch b of tile t, whose list starts at `start`, are at slot
// start / 64 + t + b (unique for lists that follow each other in tile order,
// as the binning writes them) times the tile's band count.  The backward
// walks only the marked entries and bands.
__host__ __device__ inline int64_t hit_mask_slot(int64_t start, int tile, int64_t batch) {
  return (start >> 6) + tile + batch;
}
__host__ __device__ inline int tile_bands(int tile_size) {
  return tile_size * tile_size >= 64 ? tile_size * tile_size / 64 : 1;
}
__host__ __device__ inline int64_t hit_mask_words(int64_t num_intersections, int num_tiles,
                                                  int tile_size) {
  return (num_intersections / 64 + num_tiles + 2) * tile_bands(tile_size);
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

// Per-Gaussian tile rectangle packed in 32 bits (grids of at most
// kMaxAxisTiles x kMaxAxisTiles tiles): x0 | (width - 1) << 8 | y0 << 16 |
// (height - 1) << 24, or kNoRect for a Gaussian without intersections.  The
// projection writes them (gs_project_and_count's tile_rects) and the
// row/column binning reads them: the 4 MB array for 1M Gaussians stays cache
// resident, so the depth-ordered passes gather 4 B from it instead of 16 B
// rectangles and 4 B counts from separate lines.
constexpr int kMaxAxisTiles = 256;
constexpr uint32_t kNoRect = 0xFFFFFFFFu;  // width 256 at x0 = 255 cannot occur

__host__ __device__ __forceinline__ uint32_t pack_rect(int x0, int w, int y0, int h) {
  return uint32_t(x0) | (uint32_t(w - 1) << 8) | (uint32_t(y0) << 16) | (uint32_t(h - 1) << 24);
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
