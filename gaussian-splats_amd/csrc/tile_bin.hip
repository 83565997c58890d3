// Row-bucketed tile binning for grids of at most 256 x 256 tiles.
//
// Produces exactly the sorted Gaussian ids and per-tile ranges of a stable sort
// of the reference keys tile_id << 32 | depth bits (intersections.py:10-88,
// torch.py:254-287), like gs_emit_tiles + gs_sort_tiles, while moving about a
// third of their bytes: every Gaussian covers a rectangle of tiles, so
//  1. tables: corners of the rectangles in a 2-D difference array give, after
//     a 2-D prefix sum, every tile's intersection count, hence the ranges and
//     the start of every (row, column) bucket; a 1-D difference array gives
//     the number of Gaussians covering each tile row.  No key histograms.
//  2. pass A: the depth-ordered Gaussians are expanded into one entry per
//     covered tile row and bucketed stably by row (the row list: Gaussian id,
//     first column and width per entry; about 5x fewer entries than
//     intersections).
//  3. a scan of the widths over the row list gives each row entry's first
//     position in row-major intersection order.
//  4. pass B: each row entry is expanded into its columns and bucketed stably
//     by column inside its row, straight to start(tile) + rank; only the
//     Gaussian id is written.
// Inside a tile the entries keep row-list order, which is depth order (ties by
// index), so the result is the stable (tile, depth bits, index) order.
//
// Both passes are onesweep-style (onesweep.h): ticket-ordered workgroups of
// kTile items, wave ranking by ballots, decoupled look-back for the per-digit
// offsets (pass B's chains restart at each row), reorder in LDS, coalesced
// stores.  Items are generated in registers from the owner of each position
// (marked in LDS from the scanned offsets and spread by a prefix maximum), so the expanded
// entries are never written before they are placed.
#include "block_scan.h"
#include "common.h"
#include "onesweep.h"
#include "radix.h"

namespace gs {
namespace {

using sweep::kItems;
constexpr int kSeg = kTile / 4;  // items per wave
// Rectangle tables at most this many words are accumulated in LDS first.
constexpr int kPrivateTableWords = 12288;

// ---------------------------------------------------------------------------
// Tables.
// ---------------------------------------------------------------------------

// Rectangle [x0, x1) x [y0, y1) of a packed tile rectangle, clamped to the
// grid (inside it when it comes from the projection; clamped so that no other
// input indexes out of the tables); false for kNoRect or an empty one.
__device__ __forceinline__ bool unpack_rect(uint32_t r, int tw, int th, int& x0, int& x1, int& y0,
                                            int& y1) {
  if (r == kNoRect) return false;
  x0 = min(int(r & 0xFFu), tw);
  x1 = min(x0 + int((r >> 8) & 0xFFu) + 1, tw);
  y0 = min(int((r >> 16) & 0xFFu), th);
  y1 = min(y0 + int(r >> 24) + 1, th);
  return x1 > x0 && y1 > y0;
}

// Packed rectangles from bounds [N, 2, 2] and counts (pack_rect; kNoRect for
// Gaussians without intersections), for callers that have the projection's
// bounds rather than its tile_rects output.
__global__ __launch_bounds__(256) void pack_rects_kernel(const int4* __restrict__ bounds,
                                                         const int32_t* __restrict__ counts,
                                                         int64_t n, int tw, int th,
                                                         uint32_t* __restrict__ rects) {
  const int64_t g = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (g >= n) return;
  const int4 b = bounds[g];
  const int x0 = min(max(b.x, 0), tw), x1 = min(max(b.y, 0), tw);
  const int y0 = min(max(b.z, 0), th), y1 = min(max(b.w, 0), th);
  rects[g] = counts[g] > 0 && x1 > x0 && y1 > y0 ? pack_rect(x0, x1 - x0, y0, y1 - y0) : kNoRect;
}

// Zeroes `words` 32-bit words at p (16-byte aligned): 16-byte stores over
// grid-stride rounds, then the last words.
__global__ __launch_bounds__(256) void zero_kernel(uint32_t* __restrict__ p, int64_t words) {
  const int64_t quads = words >> 2;
  const int64_t stride = int64_t(gridDim.x) * 256;
  uint4* q = reinterpret_cast<uint4*>(p);
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < quads; i += stride)
    q[i] = make_uint4(0u, 0u, 0u, 0u);
  if (blockIdx.x == 0 && int64_t(threadIdx.x) < (words & 3)) p[(quads << 2) + threadIdx.x] = 0u;
}

// Corners of each counted Gaussian's rectangle [x0, x1) x [y0, y1) in the 2-D
// difference array diff2 (th + 1 rows of pitch tw + 1) and ends of its rows in
// the 1-D difference array rowdiff (th + 1).  Grids whose tables fit LDS: each
// workgroup accumulates them there and adds them to the global ones once.
__global__ __launch_bounds__(256) void rect_diff_kernel(const uint32_t* __restrict__ rects,
                                                        int64_t n, int tw, int th,
                                                        int32_t* __restrict__ diff2,
                                                        int32_t* __restrict__ rowdiff) {
  extern __shared__ int32_t lds[];
  const int pitch = tw + 1;
  const int words = (th + 1) * pitch;
  int32_t* t2 = lds;
  int32_t* tr = lds + words;
  for (int i = threadIdx.x; i < words; i += 256) t2[i] = 0;
  for (int i = threadIdx.x; i <= th; i += 256) tr[i] = 0;
  __syncthreads();
  // Eight Gaussians per thread are loaded before their atomics are issued.
  constexpr int kBatch = 8;
  const int64_t stride = int64_t(gridDim.x) * 256;
  for (int64_t g0 = int64_t(blockIdx.x) * 256 + threadIdx.x; g0 < n; g0 += kBatch * stride) {
    uint32_t rect[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int64_t g = g0 + i * stride;
      rect[i] = g < n ? rects[g] : kNoRect;
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      int x0, x1, y0, y1;
      if (unpack_rect(rect[i], tw, th, x0, x1, y0, y1)) {
        atomicAdd(&t2[y0 * pitch + x0], 1);
        atomicAdd(&t2[y0 * pitch + x1], -1);
        atomicAdd(&t2[y1 * pitch + x0], -1);
        atomicAdd(&t2[y1 * pitch + x1], 1);
        atomicAdd(&tr[y0], 1);
        atomicAdd(&tr[y1], -1);
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < words; i += 256)
    if (t2[i]) atomicAdd(&diff2[i], t2[i]);
  for (int i = threadIdx.x; i <= th; i += 256)
    if (tr[i]) atomicAdd(&rowdiff[i], tr[i]);
}

// The same tables for grids whose difference array does not fit LDS.  Each
// workgroup takes a contiguous chunk of Gaussians, finds the window of tile
// corners its rectangles touch (first read of the chunk) and, when that window
// fits LDS, accumulates the corners there and adds the window to diff2 once
// (second read); otherwise its corners go to diff2 directly.  Chunks of a
// multi-view mosaic lie in one view (or two), whose window is that view's
// block of tiles.
__global__ __launch_bounds__(256) void rect_diff_window_kernel(const uint32_t* __restrict__ rects,
                                                               int64_t n, int64_t chunk, int tw,
                                                               int th, int32_t* __restrict__ diff2,
                                                               int32_t* __restrict__ rowdiff) {
  extern __shared__ int32_t lds[];  // kPrivateTableWords window words, then th + 1 row words
  __shared__ int s_box[4];           // -x0, x1, -y0, y1 of the corner window (max-reduced)
  const int pitch = tw + 1;
  int32_t* win = lds;
  int32_t* tr = lds + kPrivateTableWords;
  const int64_t c0 = int64_t(blockIdx.x) * chunk;
  const int64_t c1 = min(n, c0 + chunk);
  for (int i = threadIdx.x; i <= th; i += 256) tr[i] = 0;
  if (threadIdx.x < 4) s_box[threadIdx.x] = INT_MIN;
  __syncthreads();

  // Clamped rectangle of Gaussian g and whether it has intersections.
  auto rect = [&](int64_t g, int& x0, int& x1, int& y0, int& y1) {
    return unpack_rect(rects[g], tw, th, x0, x1, y0, y1);
  };

  // 1. Corner window of the chunk.
  int mx0 = INT_MIN, mx1 = INT_MIN, my0 = INT_MIN, my1 = INT_MIN;
  constexpr int kBatch = 4;
  for (int64_t g0 = c0 + threadIdx.x; g0 < c1; g0 += kBatch * 256) {
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int64_t g = g0 + i * 256;
      int x0, x1, y0, y1;
      if (g < c1 && rect(g, x0, x1, y0, y1)) {
        mx0 = max(mx0, -x0);
        mx1 = max(mx1, x1);
        my0 = max(my0, -y0);
        my1 = max(my1, y1);
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    mx0 = max(mx0, __shfl_xor(mx0, o, 64));
    mx1 = max(mx1, __shfl_xor(mx1, o, 64));
    my0 = max(my0, __shfl_xor(my0, o, 64));
    my1 = max(my1, __shfl_xor(my1, o, 64));
  }
  if ((threadIdx.x & 63) == 0) {
    atomicMax(&s_box[0], mx0);
    atomicMax(&s_box[1], mx1);
    atomicMax(&s_box[2], my0);
    atomicMax(&s_box[3], my1);
  }
  __syncthreads();
  const bool any = s_box[1] != INT_MIN;
  const int wx0 = any ? -s_box[0] : 0, wy0 = any ? -s_box[2] : 0;
  const int wpitch = any ? s_box[1] - wx0 + 1 : 0;
  const int wrows = any ? s_box[3] - wy0 + 1 : 0;
  const bool in_lds = any && wpitch * wrows <= kPrivateTableWords;
  if (in_lds)
    for (int i = threadIdx.x; i < wpitch * wrows; i += 256) win[i] = 0;
  __syncthreads();

  // 2. Corners and row ends.
  for (int64_t g0 = c0 + threadIdx.x; g0 < c1; g0 += kBatch * 256) {
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int64_t g = g0 + i * 256;
      if (g >= c1) continue;
      int x0, x1, y0, y1;
      if (rect(g, x0, x1, y0, y1)) {
        if (in_lds) {
          const int a0 = (y0 - wy0) * wpitch - wx0, a1 = (y1 - wy0) * wpitch - wx0;
          atomicAdd(&win[a0 + x0], 1);
          atomicAdd(&win[a0 + x1], -1);
          atomicAdd(&win[a1 + x0], -1);
          atomicAdd(&win[a1 + x1], 1);
        } else {
          atomicAdd(&diff2[y0 * pitch + x0], 1);
          atomicAdd(&diff2[y0 * pitch + x1], -1);
          atomicAdd(&diff2[y1 * pitch + x0], -1);
          atomicAdd(&diff2[y1 * pitch + x1], 1);
        }
        atomicAdd(&tr[y0], 1);
        atomicAdd(&tr[y1], -1);
      }
    }
  }
  __syncthreads();
  if (in_lds) {
    for (int i = threadIdx.x; i < wpitch * wrows; i += 256) {
      const int v = win[i];
      if (v) {
        const int r = i / wpitch;
        atomicAdd(&diff2[(wy0 + r) * pitch + wx0 + (i - r * wpitch)], v);
      }
    }
  }
  for (int i = threadIdx.x; i <= th; i += 256)
    if (tr[i]) atomicAdd(&rowdiff[i], tr[i]);
}

// One workgroup.  Tile counts = 2-D prefix of diff2; ranges[t] = [start,
// start + count) in row-major tile order; per row y: row_e[y] = first
// intersection, row_a[y] = first row-list entry, row_blk[y] = first pass-B
// workgroup; entry th of each holds the total.  totals = {intersections,
// row-list entries, pass-B workgroups, 0}.  With LDS_TABLE the th x (tw + 1)
// table is staged in LDS (dynamic shared memory), so the dependent prefix
// steps run at LDS latency; ranges are written once, after the row starts
// are known.
template <bool LDS_TABLE, int NT = 256>
__global__ __launch_bounds__(NT) void tables_kernel(int32_t* __restrict__ diff2,
                                                     const int32_t* __restrict__ rowdiff, int tw,
                                                     int th, int64_t* __restrict__ ranges,
                                                     uint32_t* __restrict__ row_a,
                                                     uint32_t* __restrict__ row_e,
                                                     uint32_t* __restrict__ row_blk,
                                                     int64_t* __restrict__ totals) {
  extern __shared__ int32_t tab_lds[];
  __shared__ int64_t s_row[kMaxAxisTiles];
  constexpr int NW = NT / 64;
  __shared__ int64_t scratch[NW];
  const int pitch = tw + 1;
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  int32_t* tab = LDS_TABLE ? tab_lds : diff2;
  if (LDS_TABLE) {
    for (int i = threadIdx.x; i < th * pitch; i += NT) tab[i] = diff2[i];
    __syncthreads();
  }

  // 1. Column prefix over the rows (thread x), in place.
  for (int x = threadIdx.x; x < tw; x += NT) {
    int32_t acc = 0;
    for (int y0 = 0; y0 < th; y0 += 8) {
      int32_t v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = y0 + i < th ? tab[(y0 + i) * pitch + x] : 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        acc += v[i];
        if (y0 + i < th) tab[(y0 + i) * pitch + x] = acc;
      }
    }
  }
  __syncthreads();

  // 2. One wave per row: count(x, y) = prefix over x of the column prefixes;
  // the exclusive prefix of the counts along the row (the tile's start in
  // its row) is stored in place and the row total in s_row.  32-bit: the
  // host requires fewer than 2^32 intersections.
  for (int y = wid; y < th; y += NW) {
    uint32_t carry = 0, start = 0;
    for (int x0 = 0; x0 < tw; x0 += 64) {
      const int x = x0 + lane;
      const uint32_t v = x < tw ? uint32_t(tab[y * pitch + x]) : 0u;
      const uint32_t c = carry + wave_inclusive_scan(v);
      const uint32_t cnt = x < tw ? c : 0u;
      const uint32_t inc = start + wave_inclusive_scan(cnt);
      if (x < tw) tab[y * pitch + x] = int32_t(inc - cnt);
      carry = __shfl(c, 63, 64);
      start = __shfl(inc, 63, 64);
    }
    if (lane == 0) s_row[y] = start;
  }
  __syncthreads();

  // 3. Row tables (thread y).
  const int y = threadIdx.x;
  const int64_t row_entries = y < th ? s_row[y] : 0;
  int64_t tot_e, tot_c, tot_a, tot_b;
  const int64_t e_start = block_exclusive_scan_waves<NW>(row_entries, scratch, tot_e);
  const int64_t rd = y < th ? int64_t(rowdiff[y]) : 0;
  // Gaussians on row y.
  const int64_t cover = block_exclusive_scan_waves<NW>(rd, scratch, tot_c) + rd;
  const int64_t a_start =
      block_exclusive_scan_waves<NW>(y < th ? cover : int64_t(0), scratch, tot_a);
  const int64_t blocks = (row_entries + kTile - 1) / kTile;
  const int64_t b_start = block_exclusive_scan_waves<NW>(blocks, scratch, tot_b);
  if (y < th) {
    row_e[y] = uint32_t(e_start);
    row_a[y] = uint32_t(a_start);
    row_blk[y] = uint32_t(b_start);
    s_row[y] = e_start;
  }
  __shared__ int64_t s_end[kMaxAxisTiles];
  if (y < th) s_end[y] = e_start + row_entries;
  if (threadIdx.x == 0) {
    row_e[th] = uint32_t(tot_e);
    row_a[th] = uint32_t(tot_a);
    row_blk[th] = uint32_t(tot_b);
    totals[0] = tot_e;
    totals[1] = tot_a;
    totals[2] = tot_b;
  }
  __syncthreads();

  // 4. Ranges: row start + start in the row; a tile ends where the next tile
  // of its row starts (the last one at the row's end).  totals[3] = tiles
  // with a non-empty list (the compositing launch shape depends on it) in
  // the low 32 bits, the longest list (capped at 2^31 - 1; whether the
  // compositing walk records checkpoints depends on it) in the high 32.
  const int64_t num_tiles = int64_t(tw) * th;
  int64_t active = 0;
  int64_t longest = 0;
  for (int64_t t = threadIdx.x; t < num_tiles; t += NT) {
    const int ty = int(t / tw), tx = int(t - int64_t(ty) * tw);
    const int64_t begin = s_row[ty] + uint32_t(tab[ty * pitch + tx]);
    const int64_t end = tx + 1 < tw ? s_row[ty] + uint32_t(tab[ty * pitch + tx + 1]) : s_end[ty];
    reinterpret_cast<longlong2*>(ranges)[t] = make_longlong2(begin, end);
    active += end > begin ? 1 : 0;
    longest = max(longest, end - begin);
  }
  int64_t tot_active;
  block_exclusive_scan_waves<NW>(active, scratch, tot_active);
  __syncthreads();  // scratch reused
  uint32_t l32 = uint32_t(min(longest, int64_t(0x7FFFFFFF)));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) l32 = max(l32, uint32_t(__shfl_xor(int(l32), o, 64)));
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = l32;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t mx = 0;
    for (int w = 0; w < NW; ++w) mx = max(mx, uint32_t(scratch[w]));
    totals[3] = tot_active | (int64_t(mx) << 32);
  }
}

// Row-list entry packing: first column | (width - 1) << 8 | row << 16 (grids
// of at most 256 x 256 tiles).
__device__ __forceinline__ uint32_t pack_entry(int x0, int width, int row) {
  return uint32_t(x0) | (uint32_t(width - 1) << 8) | (uint32_t(row) << 16);
}
__device__ __forceinline__ uint32_t entry_x0(uint32_t xw) { return xw & 0xFFu; }
__device__ __forceinline__ uint32_t entry_width(uint32_t xw) { return ((xw >> 8) & 0xFFu) + 1u; }
__device__ __forceinline__ uint32_t entry_row(uint32_t xw) { return (xw >> 16) & 0xFFu; }

// Row-list entries per Gaussian in depth order: its tile-row count, 0 if it
// has no intersections (from the rectangles the depth sort wrote in depth
// order: contiguous reads).
struct HeightLoad {
  const uint32_t* packed_sorted;
  __device__ static uint32_t height(uint32_t r) { return r == kNoRect ? 0u : (r >> 24) + 1u; }
  __device__ uint32_t operator()(int64_t i) const { return height(packed_sorted[i]); }
  __device__ void load4(int64_t i, uint32_t (&v)[4]) const {
    const uint4 r = *reinterpret_cast<const uint4*>(packed_sorted + i);
    v[0] = height(r.x);
    v[1] = height(r.y);
    v[2] = height(r.z);
    v[3] = height(r.w);
  }
};

// Pass-A workgroup j starts at row-list position j kTile; the Gaussian (depth
// position p) whose entries [s, s + h) contain it is recorded as
// first_a[j] = p | (starts exactly there) << 31.  h < kTile, so an entry
// range holds at most one such position.
struct HeightSink {
  uint32_t* first_a;
  uint32_t capacity;  // pass-A workgroups
  template <int M>
  __device__ void all(const int64_t (&p)[M], const uint32_t (&s)[M], const uint32_t (&h)[M],
                      int64_t n) const {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      if (p[m] >= n || h[m] == 0) continue;
      const uint32_t j = (s[m] + kTile - 1) / kTile;
      const uint32_t start = j * kTile;
      if (start < s[m] + h[m] && j < capacity)
        first_a[j] = uint32_t(p[m]) | (start == s[m] ? 0x80000000u : 0u);
    }
  }
};

// ---------------------------------------------------------------------------
// Bucketing passes.
// ---------------------------------------------------------------------------

// Largest p in [lo, hi] with offs[p] <= target, given offs[lo] <= target and
// offs non-decreasing: a 64-ary search, one ballot per round.  Wave-uniform.
__device__ int64_t wave_last_le(const uint32_t* __restrict__ offs, int64_t lo, int64_t hi,
                                uint32_t target) {
  const int lane = __lane_id();
  while (lo < hi) {
    const int64_t step = (hi - lo + 63) / 64;
    const int64_t q = min(lo + (lane + 1) * step, hi);
    const uint64_t m = __ballot(offs[q] <= target);
    const int cnt = __popcll(m);
    if (cnt == 0) {
      hi = lo + step - 1;
    } else {
      const int64_t new_lo = min(lo + cnt * step, hi);
      if (cnt < 64) hi = min(lo + (cnt + 1) * step - 1, hi);
      lo = new_lo;
    }
  }
  return lo;
}

template <int BITS, int NV>
struct BucketLds {
  uint32_t cnt[4][1 << BITS];
  uint32_t gofs[1 << BITS];
  uint32_t scratch[4];
  int64_t window[2];  // first and last owner of the workgroup's items
  uint32_t c0, nvalid, row, chain_start;
  int block;
  uint8_t dig[kTile];
  alignas(16) uint16_t own[kTile];  // owner (window index) of every position
  // Owner window (int32 offsets relative to the first item) while items are
  // generated, then the values reordered by digit.
  uint32_t val[NV * kTile];
};

// own[e] = largest k < m with rel[k] <= e, for every position e < kTile of
// the workgroup (rel[0] <= 0 < rel[1] < ... < rel[m - 1] < kTile): each owner
// k >= 1 marks its first position, and a block-wide prefix maximum over the
// positions (16 consecutive ones per thread) fills the rest.  Replaces a
// binary search per item by a few independent LDS accesses per item.
__device__ void find_owners(const int32_t* rel, int m, uint16_t* own, uint32_t* scratch) {
  uint4* own4 = reinterpret_cast<uint4*>(own);
  for (int i = threadIdx.x; i < kTile / 8; i += kBlock) own4[i] = make_uint4(0, 0, 0, 0);
  __syncthreads();
  for (int k = 1 + threadIdx.x; k < m; k += kBlock) {
    const int r = rel[k];
    if (r > 0 && r < kTile) own[r] = uint16_t(k);
  }
  __syncthreads();
  static_assert(kTile == 16 * kBlock, "16 positions per thread");
  uint4 q[2] = {own4[2 * threadIdx.x], own4[2 * threadIdx.x + 1]};
  uint32_t w[8] = {q[0].x, q[0].y, q[0].z, q[0].w, q[1].x, q[1].y, q[1].z, q[1].w};
  uint32_t run = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {  // owners never decrease: a running max
    const uint32_t lo = max(run, w[i] & 0xFFFFu);
    const uint32_t hi = max(lo, w[i] >> 16);
    w[i] = lo | (hi << 16);
    run = hi;
  }
  // Exclusive max over the threads before this one.
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const uint32_t inc = wave_inclusive_dpp(run, MaxOp{});
  if (lane == 63) scratch[wid] = inc;
  uint32_t before = dpp_read<0x138, 0xF, true>(inc);  // wave_shr:1, lane 0 reads 0
  __syncthreads();
  for (int v = 0; v < wid; ++v) before = max(before, scratch[v]);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t lo = max(before, w[i] & 0xFFFFu);
    const uint32_t hi = max(before, w[i] >> 16);
    w[i] = lo | (hi << 16);
  }
  own4[2 * threadIdx.x] = make_uint4(w[0], w[1], w[2], w[3]);
  own4[2 * threadIdx.x + 1] = make_uint4(w[4], w[5], w[6], w[7]);
  __syncthreads();
}

// Ranks the workgroup's items by digit, finds each digit's offset among the
// items of the earlier workgroups of its chain by look-back (a chain starts at
// a workgroup with chain_start), and stores the NV values of every item at
// base(d) + offset(d) + rank (below `capacity`).  Without LOOKBACK, base(d)
// is already the digit's first output position for this workgroup (status,
// b and chain_start are unused).  Items at i * 64 + lane < seg_valid of each
// wave's segment are valid; digits are below 2^BITS.
template <int BITS, int NV, bool LOOKBACK = true, typename Base>
__device__ void place_items(BucketLds<BITS, NV>& sh, const uint32_t (&dig)[kItems],
                            const uint32_t (&val)[NV][kItems], int nvalid, int b,
                            bool chain_start, Base base, uint64_t* __restrict__ status,
                            uint32_t* __restrict__ err, uint32_t* const (&out)[NV],
                            uint32_t capacity) {
  constexpr int D = 1 << BITS;
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int seg_valid = nvalid - wid * kSeg;
  uint32_t rank[kItems];
  if (nvalid == kTile)
    sweep::rank_items<BITS, true>(dig, seg_valid, sh.cnt[wid], rank);
  else
    sweep::rank_items<BITS, false>(dig, seg_valid, sh.cnt[wid], rank);
  __syncthreads();

  uint32_t tot = 0, c0 = 0, c1 = 0, c2 = 0;
  if (threadIdx.x < D) {
    c0 = sh.cnt[0][threadIdx.x];
    c1 = sh.cnt[1][threadIdx.x];
    c2 = sh.cnt[2][threadIdx.x];
    tot = c0 + c1 + c2 + sh.cnt[3][threadIdx.x];
  }
  uint32_t all;
  const uint32_t local_start = block_exclusive_scan(tot, sh.scratch, all);
  if (threadIdx.x < D) {
    const int d = threadIdx.x;
    // Wave w's items of digit d start at cnt[w][d] in the reordered tile.
    sh.cnt[0][d] = local_start;
    sh.cnt[1][d] = local_start + c0;
    sh.cnt[2][d] = local_start + c0 + c1;
    sh.cnt[3][d] = local_start + c0 + c1 + c2;
    uint64_t excl = 0;
    if constexpr (LOOKBACK) {
      uint64_t* mine = status + int64_t(b) * D + d;
      sweep::store_status(
          mine, (chain_start ? sweep::kFlagPrefix : sweep::kFlagAggregate) | uint64_t(tot));
      if (!chain_start) {
        excl = sweep::look_back(status, D, b, d, err);
        sweep::store_status(mine, sweep::kFlagPrefix | (excl + tot));
      }
    }
    // Output position of reordered item j of digit d: gofs[d] + j (mod 2^32).
    sh.gofs[d] = base(d) + uint32_t(excl) - local_start;
  }
  __syncthreads();

#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    if (i * 64 + lane < seg_valid) {
      const uint32_t d = dig[i];
      const uint32_t pos = sh.cnt[wid][d] + rank[i];
      sh.dig[pos] = uint8_t(d);
#pragma unroll
      for (int v = 0; v < NV; ++v) sh.val[v * kTile + pos] = val[v][i];
    }
  }
  __syncthreads();

  for (int j = threadIdx.x; j < nvalid; j += kBlock) {
    const uint32_t d = sh.dig[j];
    const uint32_t o = sh.gofs[d] + uint32_t(j);
    if (o < capacity) {  // always true for tables and lists built by this file
#pragma unroll
      for (int v = 0; v < NV; ++v) out[v][o] = sh.val[v * kTile + j];
    }
  }
}

// Loads the owner window [first, last] of a workgroup: rel[k] = start of
// owner first + k minus the workgroup's first position.  The span is at most
// kTile because every owner covers at least one position (Gaussians without
// intersections sort last, entries have width >= 1); a larger one, only
// possible from inconsistent inputs, is clamped and flagged.
__device__ int load_window(const uint32_t* __restrict__ offs, int64_t first, int64_t last,
                           uint32_t c0, int32_t* rel, uint32_t* err) {
  const int64_t span = last - first + 1;
  if (span > kTile && threadIdx.x == 0) atomicOr(err, kDeviceFlagWindow);
  const int m = int(min(max(span, int64_t(1)), int64_t(kTile)));
  // All of the thread's loads are issued before the first store (indices
  // clamped into the window, so every load is in bounds), for the window's
  // rounds of kBlock owners only.
  const int rounds = (m + kBlock - 1) / kBlock;  // workgroup-uniform
  uint32_t v[kTile / kBlock];
#pragma unroll
  for (int j = 0; j < kTile / kBlock; ++j)
    if (j < rounds) v[j] = offs[first + min(int(threadIdx.x) + j * kBlock, m - 1)];
#pragma unroll
  for (int j = 0; j < kTile / kBlock; ++j) {
    if (j >= rounds) break;
    const int k = int(threadIdx.x) + j * kBlock;
    if (k < m) rel[k] = int32_t(v[j] - c0);
  }
  __syncthreads();
  return m;
}

// Look-back value of the row pass for one (workgroup, tile row): its number
// of row-list entries in the low kRowCountBits bits and their intersections
// (the sum of their widths) above.  Sums along the chain stay exact while a
// row holds fewer than 2^kRowCountBits entries (the host requires fewer
// Gaussians) and fewer than 2^36 intersections (the intersection total is
// below 2^32).
constexpr int kRowCountBits = 26;
// Digits of the depth sort: up to 8 bits.  Keys remapped to 27 bits sort in
// four passes of 7, 7, 7 and 6 bits, each a few percent faster than a pass of
// 8 bits over the raw keys (fewer buckets per workgroup; three passes of 9
// bits were slower in total: 512 buckets scatter each workgroup's output
// into runs of ~8 keys).
constexpr int kDepthDigitBits = 8;
constexpr uint64_t kRowCountMask = (uint64_t(1) << kRowCountBits) - 1;

// Per-row state of a pass-A workgroup beside its bucketing arrays.
template <int BITS>
struct RowLds {
  BucketLds<BITS, 2> b;
  uint32_t wsum[1 << BITS];    // intersections of the workgroup's items of row d
  uint32_t wstart[1 << BITS];  // intersections of the workgroup's items before row d's first
  uint32_t wofs[1 << BITS];    // W of reordered item j of row d = wofs[d] + its prefix
  uint32_t e0[1 << BITS], e1[1 << BITS], blk[1 << BITS], a1[1 << BITS];  // row tables
  uint32_t waves[kItems][4];   // per round of kBlock items: each wave's sum of widths
};

// Pass A: row-list entries [b kTile, b kTile + kTile) of the depth-ordered
// expansion (Gaussian order[p] owns entries [offs[p], offs[p + 1]), one per
// covered tile row), bucketed by tile row.  The first owner comes from
// first_a (recorded by the height scan), the last one from the next
// workgroup's first owner (a search for the final workgroup).  Reads the
// packed rectangles in depth order; writes each entry's Gaussian id, packed
// first column / width / row, and W: the position of its first intersection
// in row-major intersection order (row_e[row] + the widths of the row's
// earlier entries).  The look-back carries each row's entry count and width
// sum together, so W needs no scan of its own.  The entry whose
// intersections hold a pass-B workgroup's first position records that
// workgroup's metadata
//   info[blk] = {entry | (starts exactly there) << 31, first position,
//                row | item count << 8 | (first of its row) << 31,
//                last row-list entry of the row}.
template <int BITS>
__global__ __launch_bounds__(kBlock) void row_bucket_kernel(
    const uint32_t* __restrict__ packed_sorted, const int32_t* __restrict__ order,
    const uint32_t* __restrict__ offs, const uint32_t* __restrict__ first_a, int64_t n,
    uint32_t entries, int th, const uint32_t* __restrict__ row_a,
    const uint32_t* __restrict__ row_e, const uint32_t* __restrict__ row_blk,
    const int64_t* __restrict__ totals, uint32_t blocks_b, uint32_t* __restrict__ out_g,
    uint32_t* __restrict__ out_xw, uint32_t* __restrict__ out_w, uint4* __restrict__ info,
    uint64_t* __restrict__ status, uint32_t* __restrict__ ticket, uint32_t* __restrict__ err) {
  constexpr int D = 1 << BITS;
  static_assert(D <= kBlock, "one row per thread");
  __shared__ RowLds<BITS> L;
  BucketLds<BITS, 2>& sh = L.b;
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  // Sizes from the host must be the plan's; otherwise every workgroup leaves
  // (none waits on another) and the error flag is set.
  if (totals[1] != int64_t(entries) || offs[n] != entries || totals[2] != int64_t(blocks_b)) {
    if (threadIdx.x == 0) atomicOr(err, kDeviceFlagSizes);
    return;
  }
  if (threadIdx.x == 0) sh.block = int(atomicAdd(ticket, 1u));
  for (int d = threadIdx.x; d < 4 * D; d += kBlock) (&sh.cnt[0][0])[d] = 0;
  {
    // Row tables (entry th of each holds the totals; rows at or past th
    // hold no items).
    const int d = threadIdx.x;
    if (d < D) {
      L.wsum[d] = 0;
      const bool row = d < th;
      L.e0[d] = row ? row_e[d] : 0u;
      L.e1[d] = row ? row_e[d + 1] : 0u;
      L.blk[d] = row ? row_blk[d] : 0u;
      L.a1[d] = row ? row_a[d + 1] : 0u;
    }
  }
  __syncthreads();
  const int b = sh.block;
  const int nblocks = int((int64_t(entries) + kTile - 1) / kTile);
  const uint32_t c0 = uint32_t(b) * kTile;
  const int nvalid = int(min(uint32_t(kTile), entries - c0));
  if (threadIdx.x == 0) {
    sh.window[0] = first_a[b] & 0x7FFFFFFFu;
    if (b + 1 < nblocks) {
      const uint32_t nf = first_a[b + 1];
      sh.window[1] = int64_t(nf & 0x7FFFFFFFu) - int64_t(nf >> 31);
    }
  }
  if (b + 1 == nblocks && wid == 0) {
    const int64_t p = wave_last_le(offs, 0, n - 1, c0 + uint32_t(nvalid - 1));
    if (lane == 0) sh.window[1] = p;
  }
  __syncthreads();
  const int64_t p_first = sh.window[0];
  int32_t* rel = reinterpret_cast<int32_t*>(sh.val);
  const int m = load_window(offs, p_first, sh.window[1], c0, rel, err);
  find_owners(rel, m, sh.own, sh.scratch);

  uint32_t dig[kItems];
  uint32_t g_id[kItems], xw[kItems];
  // Every position has an owner in [0, m) (the running maximum starts at 0),
  // so all gathers are in bounds: they are issued unconditionally and
  // together (the ids and the rectangles are both in depth order: one round
  // trip for the whole thread).
  int kk[kItems];
  int g[kItems];
  uint32_t r[kItems];
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    kk[i] = sh.own[wid * kSeg + i * 64 + lane];
    g[i] = order[p_first + kk[i]];
    r[i] = packed_sorted[p_first + kk[i]];
  }
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int e = wid * kSeg + i * 64 + lane;
    const uint32_t ty = (((r[i] >> 16) & 0xFFu) + uint32_t(e - rel[kk[i]])) & (D - 1u);
    dig[i] = e < nvalid ? ty : 0u;
    g_id[i] = uint32_t(g[i]);
    xw[i] = (r[i] & 0xFFFFu) | (ty << 16);  // first column, width - 1, row
  }
  // Each row's intersections in this workgroup, for the look-back value
  // (published right after the ranking; the per-item prefixes follow).
#pragma unroll
  for (int i = 0; i < kItems; ++i)
    if (wid * kSeg + i * 64 + lane < nvalid) atomicAdd(&L.wsum[dig[i]], entry_width(xw[i]));

  // 1. Stable rank by row within each wave; the rows' local starts.
  const int seg_valid = nvalid - wid * kSeg;
  uint32_t rank[kItems];
  if (nvalid == kTile)
    sweep::rank_items<BITS, true>(dig, seg_valid, sh.cnt[wid], rank);
  else
    sweep::rank_items<BITS, false>(dig, seg_valid, sh.cnt[wid], rank);
  __syncthreads();
  uint32_t tot = 0, n0 = 0, n1 = 0, n2 = 0;
  if (threadIdx.x < D) {
    n0 = sh.cnt[0][threadIdx.x];
    n1 = sh.cnt[1][threadIdx.x];
    n2 = sh.cnt[2][threadIdx.x];
    tot = n0 + n1 + n2 + sh.cnt[3][threadIdx.x];
  }
  uint32_t all;
  const uint32_t local_start = block_exclusive_scan(tot, sh.scratch, all);
  // The look-back value: (entries, intersections) of row d in this workgroup,
  // published at once so that later workgroups can walk past this one.
  const uint64_t value =
      threadIdx.x < D ? uint64_t(tot) | (uint64_t(L.wsum[threadIdx.x]) << kRowCountBits) : 0u;
  if (threadIdx.x < D) {
    const int d = threadIdx.x;
    // Wave w's items of row d start at cnt[w][d] in the reordered tile.
    sh.cnt[0][d] = local_start;
    sh.cnt[1][d] = local_start + n0;
    sh.cnt[2][d] = local_start + n0 + n1;
    sh.cnt[3][d] = local_start + n0 + n1 + n2;
    sweep::store_status(status + int64_t(b) * D + d,
                        (b == 0 ? sweep::kFlagPrefix : sweep::kFlagAggregate) | value);
  }
  __syncthreads();

  // 2. Reorder by row in LDS.
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    if (i * 64 + lane < seg_valid) {
      const uint32_t pos = sh.cnt[wid][dig[i]] + rank[i];
      sh.dig[pos] = uint8_t(dig[i]);
      sh.val[pos] = g_id[i];
      sh.val[kTile + pos] = xw[i];
    }
  }
  __syncthreads();

  // 3. Widths of the reordered items: item j = threadIdx.x + i kBlock of this
  // thread (the store layout below); wl[i] = the widths of the items before
  // it.  One wave scan per round, then the earlier rounds' and waves' sums.
  uint32_t wl[kItems], wv[kItems];
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int j = int(threadIdx.x) + i * kBlock;
    wv[i] = j < nvalid ? entry_width(sh.val[kTile + j]) : 0u;
    const uint32_t inc = wave_inclusive_dpp(wv[i], AddOp{});
    if (lane == 63) L.waves[i][wid] = inc;
    wl[i] = inc - wv[i];
  }
  __syncthreads();
  {
    uint32_t before = 0;  // widths of the earlier rounds
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
      const uint32_t s0 = L.waves[i][0], s1 = L.waves[i][1], s2 = L.waves[i][2],
                     s3 = L.waves[i][3];
      wl[i] += before + (wid > 0 ? s0 : 0u) + (wid > 1 ? s1 : 0u) + (wid > 2 ? s2 : 0u);
      before += s0 + s1 + s2 + s3;
    }
  }
  // A row's items are contiguous: its first item records the widths before
  // it.
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int j = int(threadIdx.x) + i * kBlock;
    if (j < nvalid) {
      const uint32_t d = sh.dig[j];
      if (j == 0 || sh.dig[j - 1] != d) L.wstart[d] = wl[i];
    }
  }
  __syncthreads();

  // 4. Look-back along the rows' chains: (entries, intersections) of the
  // earlier workgroups.
  if (threadIdx.x < D) {
    const int d = threadIdx.x;
    uint64_t* mine = status + int64_t(b) * D + d;
    uint64_t excl = 0;
    if (b > 0) {
      excl = sweep::look_back(status, D, b, d, err);
      sweep::store_status(mine, sweep::kFlagPrefix | (excl + value));
    }
    // Output position of reordered item j of row d: gofs[d] + j (mod 2^32).
    sh.gofs[d] = (d <= th ? row_a[d] : 0u) + uint32_t(excl & kRowCountMask) - local_start;
    if (tot) L.wofs[d] = L.e0[d] + uint32_t(excl >> kRowCountBits) - L.wstart[d];
  }
  __syncthreads();

  // 5. Stores, and the metadata of the pass-B workgroups whose first
  // position an item's intersections hold (widths are below kTile, so at
  // most one).
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int j = int(threadIdx.x) + i * kBlock;
    if (j >= nvalid) break;
    const uint32_t d = sh.dig[j];
    const uint32_t o = sh.gofs[d] + uint32_t(j);
    if (o >= entries) continue;  // never for tables and lists built by this file
    const uint32_t xwj = sh.val[kTile + j];
    const uint32_t w = L.wofs[d] + wl[i];
    out_g[o] = sh.val[j];
    out_xw[o] = xwj;
    out_w[o] = w;
    const uint32_t rel_w = w - L.e0[d];
    const uint32_t kb = (rel_w + kTile - 1) / kTile;
    const uint32_t start = kb * kTile;
    if (start < rel_w + wv[i] && L.blk[d] + kb < blocks_b) {
      const uint32_t first = L.e0[d] + start;
      const uint32_t count = min(uint32_t(kTile), L.e1[d] - first);
      info[L.blk[d] + kb] = make_uint4(o | (start == rel_w ? 0x80000000u : 0u), first,
                                       d | (count << 8) | (kb == 0 ? 0x80000000u : 0u),
                                       L.a1[d] - 1u);
    }
  }
}

// Pass B's workgroups: workgroup b covers intersections [c0, c0 + count) of
// one tile row (metadata info[b] recorded by pass A); row-list entry
// k of the row owns positions [W[k], W[k] + width) and expands into its
// columns.  Pass B buckets every intersection by column inside its row in
// three launches instead of one chained pass: counts per (workgroup, column),
// a scan of them along each row's workgroups, then the placement.  A row of
// config 4 has ~1200 workgroups, and a look-back along that chain kept each
// workgroup waiting ~14 of its 25 us.

// The owner window [first, last] of workgroup b and its first position,
// count and row.
struct PassBWindow {
  int64_t first, last;
  uint32_t c0, nvalid, row;
};
__device__ __forceinline__ PassBWindow pass_b_window(const uint4* __restrict__ info, int64_t b,
                                                     int64_t blocks) {
  const uint4 me = info[b];
  PassBWindow w;
  w.row = me.z & 0xFFu;
  w.first = me.x & 0x7FFFFFFFu;
  w.last = me.w;  // last entry of the row, unless the next workgroup shares it
  if (b + 1 < blocks) {
    const uint4 next = info[b + 1];
    if ((next.z & 0xFFu) == w.row && !(next.z >> 31))
      w.last = int64_t(next.x & 0x7FFFFFFFu) - int64_t(next.x >> 31);
  }
  w.c0 = me.y;
  w.nvalid = (me.z >> 8) & 0x1FFFu;
  // Uniform over the workgroup: kept in scalar registers.
  auto uni32 = [](uint32_t v) { return uint32_t(__builtin_amdgcn_readfirstlane(int(v))); };
  auto uni64 = [&](int64_t v) {
    return int64_t(uint64_t(uni32(uint32_t(v))) | (uint64_t(uni32(uint32_t(uint64_t(v) >> 32))) << 32));
  };
  w.first = uni64(w.first);
  w.last = uni64(w.last);
  w.c0 = uni32(w.c0);
  w.nvalid = uni32(w.nvalid);
  w.row = uni32(w.row);
  return w;
}

// Pass-B workgroups are grouped in chunks of 2^chunk_shift consecutive
// indices; the part of tile row y inside chunk k has the sums slot k + y
// (unique: a later row's workgroups all follow an earlier row's).  A chunk
// is about 1/32 of a tile row's workgroups, 16 to 64: the scan walks a
// chunk's workgroups in turn and, per row, the sums of the row's earlier
// chunks (config 3, ~80 workgroups per row: scan 16.2 -> 8.7 us with chunks
// of 16 instead of 64; config 4, ~1200: 64.8 -> 61.3 us with 32).
__host__ __device__ inline int chunk_shift(int64_t blocks, int th) {
  const int64_t per_row = (blocks + th - 1) / (th > 0 ? th : 1) / 32;
  int sh = 4;
  while (sh < 6 && (int64_t(1) << (sh + 1)) <= per_row) ++sh;
  return sh;
}
__host__ __device__ inline int64_t chunk_slots(int64_t blocks, int th) {
  const int sh = chunk_shift(blocks, th);
  return ((blocks + (int64_t(1) << sh) - 1) >> sh) + th + 1;
}

// Counts: every row-list entry of pass-B workgroup b's window adds +1 at the
// first column of its intersections inside [c0, c0 + count) and -1 after the
// last one, in an LDS difference array; its prefix over the columns is the
// workgroup's count per column, stored at counts[b * tw + column] and added
// to its chunk's sums (sums[((b >> cs) + row) * tw + column], zeroed
// beforehand).  The window's entries are read contiguously (no item is
// generated).  Two forms: one wave per window, kBlock / 64 windows per
// workgroup, for windows of a few hundred entries (config 4 ~360, config 3
// ~730: too few to keep a whole workgroup and its barriers busy; config 4
// 152 -> 97 us), and one workgroup per window for windows of thousands of
// entries (narrow entries, config 5: 63 us against 76 per wave).
template <int BITS>
__global__ __launch_bounds__(kBlock) void column_count_wave_kernel(
    const uint32_t* __restrict__ rl_xw, const uint32_t* __restrict__ W,
    const uint4* __restrict__ info, int tw, const int64_t* __restrict__ totals, int64_t total,
    int64_t entries, int64_t blocks, int cs, uint32_t* __restrict__ counts,
    uint32_t* __restrict__ sums, uint32_t* __restrict__ err) {
  constexpr int D = 1 << BITS;
  constexpr int kWaves = kBlock / 64;
  constexpr int kCols = (D + 63) / 64;  // columns per lane, consecutive
  constexpr int kBatch = 8;             // rounds of 64 entries whose loads are issued together
  __shared__ int32_t diff[kWaves][D + 1];
  if (totals[0] != total || totals[1] != entries || totals[2] != blocks) {
    if (threadIdx.x == 0) atomicOr(err, kDeviceFlagSizes);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int64_t b = int64_t(blockIdx.x) * kWaves + wid;
  if (b >= blocks) return;  // wave-uniform; the kernel has no workgroup barrier
  int32_t* const dw = diff[wid];
  for (int d = lane; d <= D; d += 64) dw[d] = 0;
  const PassBWindow win = pass_b_window(info, b, blocks);
  const int64_t span = win.last - win.first + 1;
  if (span > kTile && lane == 0) atomicOr(err, kDeviceFlagWindow);
  const int m = int(min(max(span, int64_t(1)), int64_t(kTile)));
  const uint32_t end = win.c0 + win.nvalid;
  // The zeros above are ordered before the marks: one wave's LDS accesses
  // complete in program order, and the fence keeps the compiler's order.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  for (int r0 = 0; r0 < m; r0 += 64 * kBatch) {  // wave-uniform
    uint32_t xw[kBatch], s0[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int e = min(r0 + j * 64 + lane, m - 1);
      xw[j] = rl_xw[win.first + e];
      s0[j] = W[win.first + e];
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if (r0 + j * 64 + lane >= m) continue;
      const uint32_t w = entry_width(xw[j]), x0 = entry_x0(xw[j]);
      const uint32_t lo = max(s0[j], win.c0), hi = min(s0[j] + w, end);
      if (lo < hi) {
        atomicAdd(&dw[min(x0 + (lo - s0[j]), uint32_t(D))], 1);
        atomicAdd(&dw[min(x0 + (hi - s0[j]), uint32_t(D))], -1);
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
  // Inclusive prefix over the columns: kCols consecutive ones per lane, then
  // the lanes' totals scanned across the wave.
  uint32_t c[kCols];
  uint32_t run = 0;
#pragma unroll
  for (int k = 0; k < kCols; ++k) {
    const int d = lane * kCols + k;
    run += d < D ? uint32_t(dw[d]) : 0u;
    c[k] = run;
  }
  const uint32_t before = wave_inclusive_scan(run) - run;
#pragma unroll
  for (int k = 0; k < kCols; ++k) {
    const int d = lane * kCols + k;
    const uint32_t cnt = before + c[k];
    if (d < tw) {
      counts[b * tw + d] = cnt;
      if (cnt) atomicAdd(&sums[((b >> cs) + win.row) * tw + d], cnt);
    }
  }
}

template <int BITS>
__global__ __launch_bounds__(kBlock) void column_count_block_kernel(
    const uint32_t* __restrict__ rl_xw, const uint32_t* __restrict__ W,
    const uint4* __restrict__ info, int tw, const int64_t* __restrict__ totals, int64_t total,
    int64_t entries, int64_t blocks, int cs, uint32_t* __restrict__ counts,
    uint32_t* __restrict__ sums, uint32_t* __restrict__ err) {
  constexpr int D = 1 << BITS;
  static_assert(D <= kBlock, "one column per thread");
  __shared__ int32_t diff[D + 1];
  __shared__ uint32_t scratch[4];
  if (totals[0] != total || totals[1] != entries || totals[2] != blocks) {
    if (threadIdx.x == 0) atomicOr(err, kDeviceFlagSizes);
    return;
  }
  for (int d = threadIdx.x; d <= D; d += kBlock) diff[d] = 0;
  const int64_t b = blockIdx.x;
  const PassBWindow win = pass_b_window(info, b, blocks);
  const int64_t span = win.last - win.first + 1;
  if (span > kTile && threadIdx.x == 0) atomicOr(err, kDeviceFlagWindow);
  const int m = int(min(max(span, int64_t(1)), int64_t(kTile)));
  // All of the thread's loads are issued before the first LDS update, for
  // the window's rounds of kBlock entries only (a window of wide entries
  // holds a few hundred: config 4 ~360, config 3 ~730).
  constexpr int J = kTile / kBlock;
  const int rounds = (m + kBlock - 1) / kBlock;  // workgroup-uniform
  uint32_t xw[J], s0[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if (j < rounds) {
      const int64_t k = win.first + min(int(threadIdx.x) + j * kBlock, m - 1);
      xw[j] = rl_xw[k];
      s0[j] = W[k];
    }
  }
  __syncthreads();
  const uint32_t end = win.c0 + win.nvalid;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if (j >= rounds) break;
    if (int(threadIdx.x) + j * kBlock >= m) continue;
    const uint32_t w = entry_width(xw[j]), x0 = entry_x0(xw[j]);
    const uint32_t lo = max(s0[j], win.c0), hi = min(s0[j] + w, end);
    if (lo < hi) {
      atomicAdd(&diff[min(x0 + (lo - s0[j]), uint32_t(D))], 1);
      atomicAdd(&diff[min(x0 + (hi - s0[j]), uint32_t(D))], -1);
    }
  }
  __syncthreads();
  const int d = threadIdx.x;
  const uint32_t v = d < D ? uint32_t(diff[d]) : 0u;
  uint32_t all;
  const uint32_t cnt = block_exclusive_scan(v, scratch, all) + v;
  if (d < tw) {
    counts[b * tw + d] = cnt;
    if (cnt) atomicAdd(&sums[((b >> cs) + win.row) * tw + d], cnt);
  }
}

// Threads per chunk of the column scan: the columns rounded up to whole
// waves (at most the workgroup), so a 256-thread workgroup scans two chunks
// of up to 128 columns, four of up to 64.
__host__ __device__ inline int column_scan_group(int tw) {
  const int g = ((tw + 63) / 64) * 64;
  return g < kBlock ? g : kBlock;
}

// Scan: the counts of chunk k's workgroups become each workgroup's first
// output position per column, in place: ranges[tile].start, plus the sums of
// the row's earlier chunks, plus the counts of the row's earlier workgroups
// in the chunk.  One workgroup per chunk, one thread per column; a chunk
// holds the ends of at most a few rows, walked in turn, and each thread's
// loads of a run of sums or counts are issued together.
__global__ __launch_bounds__(kBlock) void column_scan_kernel(
    uint32_t* __restrict__ counts, const uint32_t* __restrict__ sums,
    const uint4* __restrict__ info, const uint32_t* __restrict__ row_blk,
    const int64_t* __restrict__ ranges, int tw, int th, const int64_t* __restrict__ totals,
    int64_t total, int64_t entries, int64_t blocks, int cs) {
  // Inconsistent sizes were flagged by the count pass; nothing is read then.
  if (totals[0] != total || totals[1] != entries || totals[2] != blocks) return;
  // Groups of whole waves, one column per thread, one chunk per group: a
  // workgroup scans kBlock / column_scan_group(tw) chunks.
  const int group = column_scan_group(tw);
  const int sub = int(threadIdx.x) / group;
  const int64_t k = int64_t(blockIdx.x) * (kBlock / group) + sub;
  const int64_t nchunks = (blocks + (int64_t(1) << cs) - 1) >> cs;
  if (sub >= kBlock / group || k >= nchunks) return;  // wave-uniform: groups are whole waves
  const int first_d = int(threadIdx.x) - sub * group;
  const int64_t lo = k << cs, hi = min(lo + (int64_t(1) << cs), blocks);
  int64_t b = lo;
  while (b < hi) {
    const uint32_t y = min(uint32_t(__builtin_amdgcn_readfirstlane(int(info[b].z & 0xFFu))),
                           uint32_t(th - 1));
    // At least one workgroup per round, so the walk ends whatever the tables hold.
    const int64_t row_end = max(min(int64_t(row_blk[y + 1]), hi), b + 1);
    const int64_t k0 = int64_t(row_blk[y]) >> cs;  // the row's first chunk
    for (int d = first_d; d < tw; d += group) {
      uint32_t acc = uint32_t(ranges[2 * (int64_t(y) * tw + d)]);
      for (int64_t kk = k0; kk < k; kk += 8) {
        uint32_t c[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) c[i] = kk + i < k ? sums[(kk + i + y) * tw + d] : 0u;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc += c[i];
      }
      for (int64_t bb = b; bb < row_end; bb += 16) {
        uint32_t c[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) c[i] = bb + i < row_end ? counts[(bb + i) * tw + d] : 0u;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if (bb + i < row_end) {
            counts[(bb + i) * tw + d] = acc;
            acc += c[i];
          }
        }
      }
    }
    b = row_end;
  }
}

// Placement: each intersection of workgroup b is generated in registers from
// its owner, ranked by column within the workgroup and its Gaussian id
// stored at offsets[b * tw + column] + rank.
template <int BITS>
__global__ __launch_bounds__(kBlock) void column_bucket_kernel(
    const uint32_t* __restrict__ rl_g, const uint32_t* __restrict__ rl_xw,
    const uint32_t* __restrict__ W, const uint4* __restrict__ info, int tw,
    const uint32_t* __restrict__ offsets, const int64_t* __restrict__ totals, int64_t total,
    int64_t entries, int64_t blocks, int32_t* __restrict__ sorted_ids,
    uint32_t* __restrict__ err) {
  __shared__ BucketLds<BITS, 1> sh;
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  if (totals[0] != total || totals[1] != entries || totals[2] != blocks) {
    if (threadIdx.x == 0) atomicOr(err, kDeviceFlagSizes);
    return;
  }
  for (int d = threadIdx.x; d < 4 * (1 << BITS); d += kBlock) (&sh.cnt[0][0])[d] = 0;
  // Each XCD takes a contiguous range of workgroups: consecutive workgroups
  // of a row write adjacent runs of every column and share their windows'
  // edge entries in that XCD's L2 (config 4: 1130 -> 1106 us; the count
  // kernel was slower so mapped).
  const int b = xcd_swizzle(int(blockIdx.x), int(gridDim.x));
  const PassBWindow win = pass_b_window(info, b, blocks);
  const uint32_t c0 = win.c0;
  const int nvalid = int(win.nvalid);
  const int64_t k_first = win.first;
  int32_t* rel = reinterpret_cast<int32_t*>(sh.val);
  const int m = load_window(W, k_first, win.last, c0, rel, err);
  find_owners(rel, m, sh.own, sh.scratch);

  uint32_t dig[kItems];
  uint32_t val[1][kItems];
  // Owners lie in [0, m) for every position (see find_owners), so both
  // gathers are issued unconditionally and all together.
  int kk[kItems];
  uint32_t xw[kItems];
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    kk[i] = sh.own[wid * kSeg + i * 64 + lane];
    xw[i] = rl_xw[k_first + kk[i]];
    val[0][i] = rl_g[k_first + kk[i]];
  }
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int e = wid * kSeg + i * 64 + lane;
    const uint32_t d = (entry_x0(xw[i]) + uint32_t(e - rel[kk[i]])) & ((1u << BITS) - 1u);
    dig[i] = e < nvalid ? d : 0u;
  }
  uint32_t* const out[1] = {reinterpret_cast<uint32_t*>(sorted_ids)};
  const uint32_t* mine = offsets + int64_t(b) * tw;
  place_items<BITS, 1, false>(
      sh, dig, val, nvalid, b, true, [&](int d) { return d < tw ? mine[d] : 0u; }, nullptr,
      err, out, uint32_t(total));
}

template <int BITS>
void launch_row_bucket(unsigned blocks, const uint32_t* packed_sorted, const int32_t* order,
                       const uint32_t* offs, const uint32_t* first_a, int64_t n, uint32_t entries,
                       int th, const uint32_t* row_a, const uint32_t* row_e,
                       const uint32_t* row_blk, const int64_t* totals, uint32_t blocks_b,
                       uint32_t* out_g, uint32_t* out_xw, uint32_t* out_w, uint4* info,
                       uint64_t* status, uint32_t* ticket, uint32_t* err, hipStream_t s) {
  row_bucket_kernel<BITS><<<blocks, kBlock, 0, s>>>(packed_sorted, order, offs, first_a, n,
                                                    entries, th, row_a, row_e, row_blk, totals,
                                                    blocks_b, out_g, out_xw, out_w, info, status,
                                                    ticket, err);
}

// Mean row-list entries per pass-B window up to which column counting takes
// one wave per window (above: one workgroup per window).
constexpr int64_t kCountWaveEntries = 1024;

template <int BITS>
void launch_pass_b(unsigned blocks, const uint32_t* rl_g, const uint32_t* rl_xw,
                   const uint32_t* W, const uint4* info, int tw, int th, const uint32_t* row_blk,
                   const int64_t* ranges, const int64_t* totals, int64_t total, int64_t entries,
                   int64_t blocks_b, int32_t* sorted_ids, uint32_t* counts, uint32_t* sums,
                   uint32_t* err, hipStream_t s) {
  const int cs = chunk_shift(blocks_b, th);
  if (entries <= kCountWaveEntries * blocks_b)  // windows of kCountWaveEntries entries or fewer
    column_count_wave_kernel<BITS><<<unsigned(ceil_div(blocks_b, int64_t(kBlock / 64))), kBlock,
                                     0, s>>>(rl_xw, W, info, tw, totals, total, entries, blocks_b,
                                             cs, counts, sums, err);
  else
    column_count_block_kernel<BITS><<<blocks, kBlock, 0, s>>>(
        rl_xw, W, info, tw, totals, total, entries, blocks_b, cs, counts, sums, err);
  const int64_t chunks = ceil_div(blocks_b, int64_t(1) << cs);
  column_scan_kernel<<<unsigned(ceil_div(chunks, int64_t(kBlock / column_scan_group(tw)))), kBlock,
                       0, s>>>(counts, sums, info, row_blk, ranges, tw, th, totals, total, entries,
                               blocks_b, cs);
  column_bucket_kernel<BITS><<<blocks, kBlock, 0, s>>>(rl_g, rl_xw, W, info, tw, counts, totals,
                                                       total, entries, blocks_b, sorted_ids, err);
}

// Digit width of an axis of `tiles` tiles (at least 1 bit).
int axis_bits(int tiles) { return std::max(1, bits_for(tiles)); }

// Persistent plan (written by gs_bin_tiles_plan, read by gs_bin_tiles_emit).
struct PlanLayout {
  int32_t* order = nullptr;    // [n] depth order
  uint32_t* packed_sorted = nullptr;  // [n] the same in depth order (the sort's last pass)
  uint32_t* offs = nullptr;    // [n + 1] row-list offsets in depth order (written by emit)
  uint32_t* row_a = nullptr;   // [th + 1]
  uint32_t* row_e = nullptr;   // [th + 1]
  uint32_t* row_blk = nullptr;  // [th + 1]
  int32_t* table = nullptr;    // zeroed: diff2 [(th + 1) (tw + 1)], rowdiff [th + 1]
  int64_t table_words = 0;     // 64-bit words
  uint32_t* first_a = nullptr;  // [first_a_capacity] first owner of each pass-A workgroup
  uint32_t first_a_capacity = 0;
  void* sort_ws = nullptr;     // depth sort and height scan scratch
  size_t bytes = 0;
};

PlanLayout plan_layout(void* base, int64_t n, int tw, int th) {
  PlanLayout p;
  char* c = static_cast<char*>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* r = c ? c + off : nullptr;
    off += align_up(bytes);
    return r;
  };
  p.order = reinterpret_cast<int32_t*>(take(size_t(n) * 4));
  p.packed_sorted = reinterpret_cast<uint32_t*>(take(size_t(n) * 4));
  p.offs = reinterpret_cast<uint32_t*>(take(size_t(n + 1) * 4));
  p.row_a = reinterpret_cast<uint32_t*>(take(size_t(th + 1) * 4));
  p.row_e = reinterpret_cast<uint32_t*>(take(size_t(th + 1) * 4));
  p.row_blk = reinterpret_cast<uint32_t*>(take(size_t(th + 1) * 4));
  const int64_t table_ints = int64_t(th + 1) * (tw + 1) + (th + 1);
  p.table_words = (table_ints + 1) / 2;
  p.table = reinterpret_cast<int32_t*>(take(size_t(p.table_words) * 8));
  // Row-list entries are at most n th (every Gaussian on every row) and fewer
  // than 2^31 (checked by gs_bin_tiles_emit).
  p.first_a_capacity =
      uint32_t(ceil_div(std::min(int64_t(n) * th, int64_t(1) << 31), kTile) + 1);
  p.first_a = reinterpret_cast<uint32_t*>(take(size_t(p.first_a_capacity) * 4));
  const size_t sort_bytes = carve(nullptr, n, 4, 32, n, kDepthDigitBits, true).bytes;
  p.sort_ws = take(sort_bytes);
  p.bytes = off;
  return p;
}

// Scratch of gs_bin_tiles_emit.
struct EmitLayout {
  uint32_t* rl_g = nullptr;
  uint32_t* rl_xw = nullptr;
  uint32_t* W = nullptr;
  uint4* info = nullptr;        // [blocks B]
  uint64_t* zero = nullptr;     // statuses, then small words
  int64_t zero_words = 0;
  uint32_t* col = nullptr;      // [blocks B x tiles_w] pass-B counts, then offsets
  uint32_t* col_sums = nullptr;  // [chunk_slots x tiles_w] pass-B chunk sums (zeroed)
  uint64_t* status_a = nullptr;
  uint32_t* small = nullptr;  // ticket of pass A
  size_t bytes = 0;
};

EmitLayout emit_layout(void* base, int64_t entries, int64_t blocks_b, int tw, int th) {
  EmitLayout e;
  char* c = static_cast<char*>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* r = c ? c + off : nullptr;
    off += align_up(bytes);
    return r;
  };
  const int64_t blocks_a = ceil_div(entries, kTile);
  e.rl_g = reinterpret_cast<uint32_t*>(take(size_t(entries) * 4));
  e.rl_xw = reinterpret_cast<uint32_t*>(take(size_t(entries) * 4));
  e.W = reinterpret_cast<uint32_t*>(take(size_t(entries) * 4));
  e.info = reinterpret_cast<uint4*>(take(size_t(blocks_b + 1) * 16));
  e.col = reinterpret_cast<uint32_t*>(take(size_t(blocks_b) * size_t(tw) * 4));
  const int64_t words_a = blocks_a << axis_bits(th);
  const int64_t words_s = (chunk_slots(blocks_b, th) * tw + 1) / 2;
  e.zero_words = words_a + words_s + 4;  // + 8 small 32-bit words
  e.zero = reinterpret_cast<uint64_t*>(take(size_t(e.zero_words) * 8));
  if (e.zero) {
    e.status_a = e.zero;
    e.col_sums = reinterpret_cast<uint32_t*>(e.status_a + words_a);
    e.small = reinterpret_cast<uint32_t*>(e.status_a + words_a + words_s);
  }
  e.bytes = off;
  return e;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_grid(int tiles_w, int tiles_h) {
  GS_REQUIRE(tiles_w > 0 && tiles_h > 0, GS_ERR_INVALID_ARGUMENT, "empty tile grid");
  GS_REQUIRE(tiles_w <= kMaxAxisTiles && tiles_h <= kMaxAxisTiles, GS_ERR_UNSUPPORTED,
             "row-bucketed binning needs at most %d x %d tiles (got %d x %d)", kMaxAxisTiles,
             kMaxAxisTiles, tiles_w, tiles_h);
  return GS_OK;
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" {

GS_API size_t gs_bin_tiles_plan_bytes(int64_t n, int32_t tiles_w, int32_t tiles_h) {
  if (n < 0 || tiles_w <= 0 || tiles_h <= 0) return 0;
  return plan_layout(nullptr, n, tiles_w, tiles_h).bytes;
}

GS_API int gs_pack_tile_rects(const int32_t* bounds, const int32_t* counts, int64_t n,
                              int32_t tiles_w, int32_t tiles_h, uint32_t* tile_rects,
                              void* stream) {
  clear_error();
  GS_TRY(check_grid(tiles_w, tiles_h));
  GS_REQUIRE(n >= 0, GS_ERR_INVALID_ARGUMENT, "invalid Gaussian count");
  if (n == 0) return GS_OK;
  GS_REQUIRE(bounds && counts && tile_rects && aligned16(bounds), GS_ERR_INVALID_ARGUMENT,
             "null or misaligned pointer");
  pack_rects_kernel<<<unsigned(ceil_div(n, 256)), 256, 0, as_stream(stream)>>>(
      reinterpret_cast<const int4*>(bounds), counts, n, tiles_w, tiles_h, tile_rects);
  return check_launch("pack_tile_rects");
}

GS_API int gs_bin_tiles_plan(uint32_t* depth_keys, const uint32_t* tile_rects, int64_t n,
                             uint32_t key_base, int32_t key_bits, int32_t tiles_w,
                             int32_t tiles_h, int64_t* ranges, int64_t* totals,
                             int64_t* host_totals, void* plan, size_t plan_bytes, void* clear_buf,
                             size_t clear_bytes, void* stream) {
  clear_error();
  GS_TRY(check_grid(tiles_w, tiles_h));
  GS_REQUIRE(n >= 0, GS_ERR_INVALID_ARGUMENT, "invalid Gaussian count");
  GS_REQUIRE(key_bits >= 1 && key_bits <= 32, GS_ERR_INVALID_ARGUMENT,
             "key_bits must be in [1, 32], got %d", key_bits);
  GS_REQUIRE(n < (int64_t(1) << kRowCountBits), GS_ERR_OVERFLOW,
             "row/column bucketing takes fewer than %lld Gaussians (got %lld)",
             (long long)(int64_t(1) << kRowCountBits), (long long)n);
  GS_REQUIRE(ranges && totals && plan, GS_ERR_INVALID_ARGUMENT, "null pointer argument");
  GS_REQUIRE(aligned16(ranges), GS_ERR_INVALID_ARGUMENT, "ranges must be 16-byte aligned");
  GS_REQUIRE(n == 0 || (depth_keys && tile_rects), GS_ERR_INVALID_ARGUMENT,
             "null pointer argument");
  GS_REQUIRE(!clear_buf || (aligned16(clear_buf) && clear_bytes % 4 == 0), GS_ERR_INVALID_ARGUMENT,
             "the buffer to clear must be 16-byte aligned and a multiple of 4 bytes");
  const PlanLayout p = plan_layout(plan, n, tiles_w, tiles_h);
  GS_REQUIRE(plan_bytes >= p.bytes, GS_ERR_WORKSPACE, "plan workspace too small (%zu < %zu)",
             plan_bytes, p.bytes);
  hipStream_t s = as_stream(stream);
  uint32_t* flags = nullptr;
  GS_TRY(device_flags(s, &flags));
  // The tile tables need only the rectangles: they run on the side stream
  // while the depth sort and the row-list offset scan run on the caller's.
  // The sort's clear, histogram and first pass are enqueued first, so the
  // caller's stream has work while the host enqueues the side stream's
  // kernels; the copies of the totals (slow host calls) are enqueued last,
  // once every kernel of both streams is.  (Under the kernel trace, whose
  // launches are slower, copies enqueued before the other passes held them
  // back 30-50 us on config 3; unprofiled steps measured the same either
  // way.)
  SideFork fork;
  GS_TRY(fork_side_stream(s, fork));
  const int words = (tiles_h + 1) * (tiles_w + 1);
  auto side_work = [&]() -> int {
    sweep::clear_kernel<<<unsigned(std::max<int64_t>(1, std::min<int64_t>(256, ceil_div(p.table_words, kBlock)))),
                          kBlock, 0, fork.side>>>(reinterpret_cast<uint64_t*>(p.table),
                                                  p.table_words, nullptr, 0);
    if (n > 0) {
      const unsigned blocks = unsigned(std::min<int64_t>(256, std::max<int64_t>(1, ceil_div(n, 4096))));
      int32_t* diff2 = p.table;
      int32_t* rowdiff = p.table + words;
      if (words + tiles_h + 1 <= kPrivateTableWords) {
        rect_diff_kernel<<<blocks, 256, size_t(words + tiles_h + 1) * 4, fork.side>>>(
            tile_rects, n, tiles_w, tiles_h, diff2, rowdiff);
      } else {
        // Contiguous chunks with private corner windows (see the kernel).
        const int64_t wblocks = std::min<int64_t>(512, std::max<int64_t>(1, ceil_div(n, 16384)));
        const int64_t chunk = ceil_div(n, wblocks);
        rect_diff_window_kernel<<<unsigned(ceil_div(n, chunk)), 256,
                                  size_t(kPrivateTableWords + tiles_h + 1) * 4, fork.side>>>(
            tile_rects, n, chunk, tiles_w, tiles_h, diff2,
            rowdiff);
      }
    }
    int st = GS_OK;
    const int lds_words = tiles_h * (tiles_w + 1);
    if (lds_words <= kPrivateTableWords) {
      tables_kernel<true><<<1, 256, size_t(lds_words) * 4, fork.side>>>(
          p.table, p.table + words, tiles_w, tiles_h, ranges, p.row_a, p.row_e, p.row_blk, totals);
    } else {
      // In global memory every step waits on memory: 16 waves instead of 4
      // (config 5: 200 x 200 tiles, 330 -> 120 us).
      tables_kernel<false, 1024><<<1, 1024, 0, fork.side>>>(p.table, p.table + words, tiles_w,
                                                            tiles_h, ranges, p.row_a, p.row_e,
                                                            p.row_blk, totals);
    }
    // The caller's buffer to clear (the op's gradient accumulator), beside
    // the depth sort and before the totals: the host's wait for them, or the
    // join, orders it before anything enqueued after this call.
    if (clear_buf && clear_bytes >= 4) {
      const int64_t words = int64_t(clear_bytes / 4);
      zero_kernel<<<unsigned(std::max<int64_t>(1, std::min<int64_t>(2048, ceil_div(words, 1024)))),
                    256, 0, fork.side>>>(static_cast<uint32_t*>(clear_buf), words);
    }
    if (st == GS_OK) st = check_launch("bin_tiles_plan (tables)");
    return st;
  };
  auto copy_totals = [&]() -> int {
    int st = GS_OK;
    // The totals, then the sticky check-failure word beside them (its low
    // half; the caller keeps the high half zero).
    if (host_totals &&
        (hipMemcpyAsync(host_totals, totals, 4 * sizeof(int64_t), hipMemcpyDeviceToHost,
                        fork.side) != hipSuccess ||
         hipMemcpyAsync(host_totals + 4, flags, sizeof(uint32_t), hipMemcpyDeviceToHost,
                        fork.side) != hipSuccess)) {
      set_error("bin_tiles_plan: copy of the totals failed");
      st = GS_ERR_HIP;
    }
    return st;
  };
  int status = GS_OK;
  if (n > 0) {
    Scratch ws = carve(p.sort_ws, n, 4, 32, n, kDepthDigitBits, true);
    ws.flags = flags;
    clear(ws, s);
    // depth_keys is consumed (ping-pong buffer of the sort).
    uint32_t* sorted_keys = nullptr;
    // The packed rectangles move with the keys through every pass (a payload
    // in index order), so the last pass writes them in depth order.
    // With key_bits < 32 the sort orders min(key - key_base, 2^key_bits - 1)
    // in digits of up to kDepthDigitBits bits.
    KeyRemap remap;
    remap.on = key_bits < 32;
    remap.base = key_base;
    remap.max_bits = kDepthDigitBits;
    status = radix_sort<uint32_t, true>(depth_keys, nullptr, n, key_bits,
                                        reinterpret_cast<uint32_t*>(p.order), &sorted_keys, ws, s,
                                        tile_rects, p.packed_sorted, side_work, remap);
    // Row-list offsets in depth order, recording each pass-A workgroup's
    // first owner.
    if (status == GS_OK)
      launch_scan<uint32_t>(HeightLoad{p.packed_sorted}, n, p.offs, true, true, ws, s,
                            HeightSink{p.first_a, p.first_a_capacity});
  } else {
    status = side_work();
  }
  if (status == GS_OK) status = copy_totals();
  // Always join, also after an error; with host_totals the host waits for
  // the tables only, while the sort keeps running on the caller's stream
  // (the caller's stream then needs no wait of its own: everything enqueued
  // on it after this call follows the side stream's work).
  const int joined = join_side_stream(fork, host_totals != nullptr && status == GS_OK);
  GS_TRY(status);
  GS_TRY(joined);
  return check_launch("bin_tiles_plan");
}

GS_API size_t gs_bin_tiles_emit_bytes(int64_t n, int64_t total, int64_t row_entries,
                                      int64_t blocks, int32_t tiles_w, int32_t tiles_h) {
  if (n < 0 || total < 0 || row_entries < 0 || blocks < 0 || tiles_w <= 0 || tiles_h <= 0)
    return 0;
  return emit_layout(nullptr, row_entries, blocks, tiles_w, tiles_h).bytes;
}

GS_API int gs_bin_tiles_emit(int64_t n,
                             int32_t tiles_w, int32_t tiles_h, const int64_t* totals,
                             int64_t total, int64_t row_entries, int64_t blocks, void* plan,
                             size_t plan_bytes, const int64_t* ranges, int32_t* sorted_ids,
                             void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  GS_TRY(check_grid(tiles_w, tiles_h));
  GS_REQUIRE(n >= 0 && total >= 0 && row_entries >= 0 && blocks >= 0, GS_ERR_INVALID_ARGUMENT,
             "invalid emit arguments");
  GS_REQUIRE(n < (int64_t(1) << kRowCountBits), GS_ERR_OVERFLOW,
             "row/column bucketing takes fewer than %lld Gaussians (got %lld)",
             (long long)(int64_t(1) << kRowCountBits), (long long)n);
  GS_REQUIRE(total < (int64_t(1) << 32) - kTile && row_entries < (int64_t(1) << 31),
             GS_ERR_OVERFLOW, "too many intersections (%lld)", (long long)total);
  GS_REQUIRE(blocks >= ceil_div(total, kTile) && blocks <= ceil_div(total, kTile) + tiles_h,
             GS_ERR_INVALID_ARGUMENT, "inconsistent workgroup count");
  if (total == 0) return GS_OK;
  GS_REQUIRE(n > 0 && row_entries > 0 && blocks > 0, GS_ERR_INVALID_ARGUMENT,
             "intersections without Gaussians");
  GS_REQUIRE(totals && plan && ranges && sorted_ids && workspace, GS_ERR_INVALID_ARGUMENT,
             "null pointer argument");
  const PlanLayout p = plan_layout(plan, n, tiles_w, tiles_h);
  GS_REQUIRE(plan_bytes >= p.bytes, GS_ERR_WORKSPACE, "plan workspace too small");
  const EmitLayout e = emit_layout(workspace, row_entries, blocks, tiles_w, tiles_h);
  GS_REQUIRE(uint64_t(ceil_div(row_entries, kTile)) <= p.first_a_capacity, GS_ERR_INVALID_ARGUMENT,
             "row-list entries exceed the plan");
  GS_REQUIRE(workspace_bytes >= e.bytes, GS_ERR_WORKSPACE, "emit workspace too small (%zu < %zu)",
             workspace_bytes, e.bytes);
  hipStream_t s = as_stream(stream);
  uint32_t* err = nullptr;  // the device's sticky check-failure word
  GS_TRY(device_flags(s, &err));
  sweep::clear_kernel<<<unsigned(std::max<int64_t>(1, std::min<int64_t>(1024, ceil_div(e.zero_words, kBlock)))),
                        kBlock, 0, s>>>(e.zero, e.zero_words, nullptr, 0);
  uint32_t* ticket_a = e.small;
  const unsigned blocks_a = unsigned(ceil_div(row_entries, kTile));
  // Pass A also writes every row-list entry's position in row-major
  // intersection order and each pass-B workgroup's metadata.
  switch (axis_bits(tiles_h)) {
#define GS_ROW_CASE(B)                                                                          \
  case B:                                                                                       \
    launch_row_bucket<B>(blocks_a, p.packed_sorted, p.order, p.offs, p.first_a, n,              \
                         uint32_t(row_entries), tiles_h, p.row_a, p.row_e, p.row_blk, totals,   \
                         uint32_t(blocks), e.rl_g, e.rl_xw, e.W, e.info, e.status_a, ticket_a,  \
                         err, s);                                                               \
    break;
    GS_ROW_CASE(1) GS_ROW_CASE(2) GS_ROW_CASE(3) GS_ROW_CASE(4)
    GS_ROW_CASE(5) GS_ROW_CASE(6) GS_ROW_CASE(7) GS_ROW_CASE(8)
#undef GS_ROW_CASE
  }
  switch (axis_bits(tiles_w)) {
#define GS_COL_CASE(B)                                                                          \
  case B:                                                                                       \
    launch_pass_b<B>(unsigned(blocks), e.rl_g, e.rl_xw, e.W, e.info, tiles_w, tiles_h,          \
                     p.row_blk, ranges, totals, total, row_entries, blocks, sorted_ids, e.col,   \
                     e.col_sums, err, s);                                                       \
    break;
    GS_COL_CASE(1) GS_COL_CASE(2) GS_COL_CASE(3) GS_COL_CASE(4)
    GS_COL_CASE(5) GS_COL_CASE(6) GS_COL_CASE(7) GS_COL_CASE(8)
#undef GS_COL_CASE
  }
  return check_launch("bin_tiles_emit");
}

}  // extern "C"
