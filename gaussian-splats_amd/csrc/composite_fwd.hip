// Forward compositing: one wave64 per work item -- a whole tile, tile_size^2 /
// 64 pixels per lane, or a quarter of a heavy tile's pixel bands (the dispatch
// plan of tile_order.hip) -- front-to-back over the tile's depth-sorted list.
//
// Pixel semantics are those of kernels/rasterize/torch.py:172-225 with the
// sequential transmittance and contributor count of composite.py:44-107:
//   alpha = min(o * exp(-D/2), 0.99), zeroed below 1/255;
//   a pixel is active for an entry while (1 - T) < opacity_threshold, checked
//   before blending (as T > 1 - opacity_threshold); C += T * alpha * rgb;
//   T *= (1 - alpha) while active (as T - T alpha);
//   n_contributors = entries processed while active (the position after the
//   entry that deactivated the pixel, or the list length).
// Integer pixel coordinates (no +0.5, torch.py:157-168), black background.
//
// Each lane gathers one Gaussian record of the next 64 list entries and tests
// whether it can reach alpha >= 1/255 anywhere in the rectangle spanned by
// the wave's pixels still active (touches_rect, band_span); the wave then
// walks only the set bits of that ballot, reading each record as an LDS
// broadcast.  The tile stops as soon as no pixel is active.  With hit masks,
// each batch's ballot is stored for the backward, which then gathers only
// the entries it marks.
#include "common.h"
#include "raster_math.h"

namespace gs {
namespace {

struct CompositeArgs {
  const GsRecord* records;
  uint32_t max_id;  // last valid record index: every gathered id is clamped to it
  const int32_t* ids;
  const int64_t* ranges;
  const int32_t* items;  // dispatch plan (gs_tile_order), or nullptr: tiles in index order
  int num_items;
  bool split_all;        // without a plan: every tile split into quarters
  int width, height, tile;  // per view
  int tiles_w, num_tiles;    // of the whole mosaic
  int view_tw, view_th, cols, views;  // tiles per view, mosaic layout (one view: cols = views = 1)
  float threshold;
  // A pixel stays active while (1 - T) < threshold, i.e. T > 1 - threshold.
  float t_active;
  float* image;
  float* final_t;
  int32_t* n_contrib;
  // Checkpoints of whole-tile walks for the backward (CheckpointLayout), or
  // null counter: none.
  uint32_t* ckpt_counter;
  int32_t* ckpt_table;
  float4* ckpt_records;
  int64_t ckpt_capacity;
  // The walked batches' hit masks (hit_mask_slot), or null: none.
  uint64_t* hit_masks;
  int64_t hit_capacity;  // words
  // The backward's dispatch keys (gs_tile_order's workspace layout: per tile
  // its largest contributor count, capped at 2^16 - 1, then per tile the
  // checkpoints a backward walk crosses), written by whole-tile walks; or
  // null: none.
  uint32_t* tile_keys;
};

// One wave composites PIX pixels per lane of `tile`: the 64-pixel bands
// band0 .. band0 + PIX - 1 (all of the tile's bands for a whole-tile item, a
// quarter of them for a quarter item; every wave walks the whole list).
// With `checkpoints` (whole tiles only) the walk records the checkpoints
// described at CheckpointLayout; with HITS, every walked batch's overlap
// ballot in the hit-mask words of each of the wave's bands.
// With `write_key` (a whole-tile walk) and a.tile_keys, the tile's backward
// dispatch key and checkpoint crossings are written once its walk ends.
template <int TILE, bool ELLIPSOID, int PIX, bool HITS, bool PF = false>
__device__ __forceinline__ void composite_tile(const CompositeArgs& a, float4 (*chunk)[3],
                                               float4 (*chunk2)[3], int* ck_slots, int lane,
                                               int tile, int band0, bool checkpoints,
                                               bool write_key) {
  constexpr int NPIX = TILE * TILE;

  // Mosaic tile -> view and the tile's pixel origin inside that view.
  const int tx = tile % a.tiles_w;
  const int ty = tile / a.tiles_w;
  const int vx = tx / a.view_tw, vy = ty / a.view_th;
  const int view = vy * a.cols + vx;
  const int64_t start = a.ranges[2 * tile];
  const int64_t end = a.ranges[2 * tile + 1];
  const int list_len = int(end - start);
  write_key = write_key && a.tile_keys;
  if (view >= a.views) {  // an empty slot of the mosaic's last row
    if (write_key && lane == 0) {
      a.tile_keys[tile] = 0u;
      a.tile_keys[a.num_tiles + tile] = uint32_t(checkpoint_count(start, 0, list_len));
    }
    return;
  }
  const int ox = (tx - vx * a.view_tw) * TILE, oy = (ty - vy * a.view_th) * TILE;
  const int64_t view_base = int64_t(view) * a.width * a.height;  // first pixel of the view

  // The lane's pixels share one column (see column_terms).
  const float pxf = float(ox + lane % TILE);
  float pyf[PIX];
  float T[PIX], cr[PIX], cg[PIX], cb[PIX];
  // A pixel is active at list position pos while pos < ncon: ncon starts at
  // the list length (0 for an inactive pixel) and becomes pos + 1 at the
  // entry that deactivates it.  No per-pixel flag is carried through the
  // walk: the comparison replaces the lane-mask merges that a loop-carried
  // flag costs in scalar instructions per entry.
  int ncon[PIX];
  const bool start_active = (1.0f - 1.0f) < a.threshold;
#pragma unroll
  for (int k = 0; k < PIX; ++k) {
    const int q = lane + 64 * (band0 + k);
    const int px = ox + (q % TILE), py = oy + (q / TILE);
    const bool valid = q < NPIX && px < a.width && py < a.height;
    pyf[k] = float(py);
    T[k] = 1.0f;
    cr[k] = cg[k] = cb[k] = 0.0f;
    ncon[k] = valid && start_active ? list_len : 0;
  }
  constexpr int kBandRows = 64 / TILE > 0 ? 64 / TILE : 1;  // tile rows per band

  bool running;
  {
    bool l = false;
#pragma unroll
    for (int k = 0; k < PIX; ++k) l |= ncon[k] > 0;
    running = __ballot(l) != 0;
  }
  constexpr int kBands = NPIX >= 64 ? NPIX / 64 : 1;  // the tile's 64-pixel bands
  // Checkpoint state (wave-uniform): crossings reached, records written (a
  // prefix of the crossings: once the pool is full every later allocation
  // fails), the walk position of the next crossing; the records' slots go to
  // the wave's ck_slots in LDS.
  constexpr int kRecord = PIX * 64;
  int ck_count = 0, ck_written = 0;
  int ck_next =
      checkpoints && checkpoint_count(start, list_len, list_len) > 0 ? checkpoint_batch(start, 1)
                                                                     : -1;
  // Crossing ck_count + 1 at list offset bpos (a batch start): record T and
  // the colour since the previous record, then restart the colour sums.
  auto checkpoint_at = [&](int bpos) {
    if (!(checkpoints && bpos == ck_next)) return;
    uint32_t slot = 0xFFFFFFFFu;
    if (lane == 0 && ck_written == ck_count) slot = atomicAdd(a.ckpt_counter, 1u);
    slot = uint32_t(__builtin_amdgcn_readfirstlane(int(slot)));
    const bool ok = ck_written == ck_count && int64_t(slot) < a.ckpt_capacity;
    const int64_t pos = checkpoint_first(start) + int64_t(ck_count) * kCheckpointEntries;
    if (lane == 0) a.ckpt_table[pos / kCheckpointEntries] = ok ? int32_t(slot) : -1;
    if (ok) {
      float4* rec = a.ckpt_records + int64_t(slot) * kRecord;
#pragma unroll
      for (int k = 0; k < PIX; ++k) {
        rec[lane + 64 * k] = make_float4(T[k], cr[k], cg[k], cb[k]);
        cr[k] = cg[k] = cb[k] = 0.0f;
      }
      if (lane == 0) ck_slots[ck_written] = int(slot);
      ++ck_written;
    }
    ++ck_count;
    ck_next = ck_count < kMaxCheckpoints ? checkpoint_batch(start, ck_count + 1) : -1;
  };
  // The overlap test's rectangle: the columns and rows of the pixels still
  // active at list offset bpos (a set that only shrinks along the walk; the
  // walk is running, so it is not empty).
  auto active_rect = [&](int bpos, float& rx0, float& rx1, float& ry0, float& ry1) {
    uint32_t cols = 0;
    int rlo = NPIX, rhi = -1;
#pragma unroll
    for (int k = 0; k < PIX; ++k) {
      const uint64_t m = __ballot(bpos < ncon[k]);
      if (m) {
        uint32_t c;
        int r0, r1;
        band_span<TILE>(m, c, r0, r1);
        cols |= c;
        rlo = min(rlo, (band0 + k) * kBandRows + r0);
        rhi = max(rhi, (band0 + k) * kBandRows + r1);
      }
    }
    rx0 = float(ox + __builtin_ctz(cols));
    rx1 = float(ox + 31 - __builtin_clz(cols));
    ry0 = float(oy + rlo);
    ry1 = float(oy + rhi);
  };
  auto stage = [&](float4 (*rows)[3], const LaneSplat& mine) {
    rows[lane][0] = make_float4(mine.u, mine.v, mine.o, mine.pa);
    rows[lane][1] = make_float4(mine.pb, mine.pc, mine.r, mine.g);
    rows[lane][2] = make_float4(mine.b, mine.cut, 0.0f, 0.0f);
  };
  // The batch's mask, the entries that can reach a pixel of the wave's bands
  // still active, stored for each of the bands (vector stores).
  auto store_hits = [&](uint64_t mask, int64_t base) {
    if constexpr (HITS) {
      const int64_t w0 = hit_mask_slot(start, tile, (base - start) >> 6) * kBands + band0;
      if (lane < PIX && w0 + lane < a.hit_capacity) a.hit_masks[w0 + lane] = mask;
    }
  };
  // Blends the kept entries of the batch at `base` (staged in `rows`) in list
  // order.  No break inside: the loop ends through its condition, which keeps
  // the walk's state out of extra mask-merging control flow.
  auto composite_batch = [&](uint64_t mask, float4 (*rows)[3], int64_t base) {
    while (mask) {
      const int j = __builtin_ctzll(mask);
      mask &= mask - 1;
      const float4 f0 = rows[j][0], f1 = rows[j][1], f2 = rows[j][2];
      Splat s;
      s.u = f0.x;
      s.v = f0.y;
      s.o = f0.z;
      s.pa = f0.w;
      s.pb = f1.x;
      s.pc = f1.y;
      s.r = f1.z;
      s.g = f1.w;
      s.bl = f2.x;
      s.cut = f2.y;
      const int pos = int(base - start) + j;
      const ColumnTerms c = column_terms(s, pxf);
      // Branch-free: a finished pixel (or a cut alpha) blends with alpha = 0,
      // which leaves its colour and T unchanged.  T (1 - alpha) = T - w.
      bool still = false;  // a pixel of the lane stays active after the entry
#pragma unroll
      for (int k = 0; k < PIX; ++k) {
        float prob;
        const float raw = raw_alpha<ELLIPSOID>(s, c, pyf[k] - s.v, prob);
        const float clamped = fminf(raw, kMaxAlpha);
        const bool live = pos < ncon[k];
        const bool take = live && clamped >= kMinAlpha;  // alpha = blend_alpha(raw) > 0
        const float alpha = take ? clamped : 0.0f;
        const float w = T[k] * alpha;
        cr[k] += w * s.r;
        cg[k] += w * s.g;
        cb[k] += w * s.bl;
        T[k] = T[k] - w;
        const bool done = live && !(T[k] > a.t_active);
        ncon[k] = done ? pos + 1 : ncon[k];
        still |= live && !done;
      }
      if (__ballot(still) == 0) {
        running = false;
        mask = 0;
      }
    }
  };

  uint32_t id = start + lane < end ? uint32_t(a.ids[start + lane]) : 0u;
  if constexpr (PF) {
    // Long lists (the checkpoint kernel), whose walks are latency bound: two
    // batches per step.  Both are tested against the rectangle of the pixels
    // active at the first one's start (for the second, a superset of its own
    // rectangle: an entry kept only by it reaches alpha >= 1/255 at no active
    // pixel and blends nothing), so the two tests' dependent chains overlap,
    // and both batches' records are requested a step ahead (ids two ahead).
    // Unconditional loads: lanes past the list read record 0, and this
    // kernel runs only with records (the host's condition for checkpoints).
    GsRecord next0 = load_record(a.records, min(id, a.max_id));
    id = start + 64 + lane < end ? uint32_t(a.ids[start + 64 + lane]) : 0u;
    GsRecord next1 = load_record(a.records, min(id, a.max_id));
    uint32_t id0 = start + 128 + lane < end ? uint32_t(a.ids[start + 128 + lane]) : 0u;
    uint32_t id1 = start + 192 + lane < end ? uint32_t(a.ids[start + 192 + lane]) : 0u;
    for (int64_t base = start; running && base < end; base += 128) {
      checkpoint_at(int(base - start));
      float rx0, rx1, ry0, ry1;
      active_rect(int(base - start), rx0, rx1, ry0, ry1);
      const int64_t e = base + lane;
      const bool second = base + 64 < end;  // wave-uniform
      LaneSplat mine0, mine1;
      bool keep0 = false, keep1 = false;
      if (e < end) {
        keep0 = touches_rect(next0, rx0, rx1, ry0, ry1);
        mine0 = lane_splat(next0);
      }
      if (e + 64 < end) {
        keep1 = touches_rect(next1, rx0, rx1, ry0, ry1);
        mine1 = lane_splat(next1);
      }
      stage(chunk, mine0);
      stage(chunk2, mine1);
      next0 = load_record(a.records, min(id0, a.max_id));
      next1 = load_record(a.records, min(id1, a.max_id));
      id0 = e + 256 < end ? uint32_t(a.ids[e + 256]) : 0u;
      id1 = e + 320 < end ? uint32_t(a.ids[e + 320]) : 0u;
      const uint64_t mask0 = __ballot(keep0), mask1 = __ballot(keep1);
      store_hits(mask0, base);
      if (second) store_hits(mask1, base + 64);
      composite_batch(mask0, chunk, base);
      if (running && second) {
        checkpoint_at(int(base + 64 - start));
        composite_batch(mask1, chunk2, base + 64);
      }
    }
  } else {
    // The ids of each batch are requested one batch ahead, once the current
    // batch's records are in LDS, so they arrive while the current batch is
    // walked and each batch waits on one dependent load (the record gather).
    for (int64_t base = start; running && base < end; base += 64) {
      checkpoint_at(int(base - start));
      float rx0, rx1, ry0, ry1;
      active_rect(int(base - start), rx0, rx1, ry0, ry1);
      const int64_t e = base + lane;
      LaneSplat mine;
      bool keep = false;
      if (e < end) {
        const GsRecord rec = load_record(a.records, min(id, a.max_id));
        keep = touches_rect(rec, rx0, rx1, ry0, ry1);
        mine = lane_splat(rec);
      }
      stage(chunk, mine);
      id = e + 64 < end ? uint32_t(a.ids[e + 64]) : 0u;
      const uint64_t mask = __ballot(keep);
      store_hits(mask, base);
      composite_batch(mask, chunk, base);
    }
  }
  // The records' colours become the colour composited after each record (a
  // suffix sum over the later records and the colour since the last one); the
  // image is the sum over all of them.  Each lane reads back its own writes.
  for (int j = checkpoints ? ck_written - 1 : -1; j >= 0; --j) {
    float4* rec = a.ckpt_records + int64_t(ck_slots[j]) * kRecord;
#pragma unroll
    for (int k = 0; k < PIX; ++k) {
      const float4 v = rec[lane + 64 * k];
      rec[lane + 64 * k] = make_float4(v.x, cr[k], cg[k], cb[k]);
      cr[k] += v.y;
      cg[k] += v.z;
      cb[k] += v.w;
    }
  }

#pragma unroll
  for (int k = 0; k < PIX; ++k) {
    const int q = lane + 64 * (band0 + k);
    const int px = ox + (q % TILE), py = oy + (q / TILE);
    if (q < NPIX && px < a.width && py < a.height) {
      const int64_t pix = view_base + int64_t(py) * a.width + px;
      a.image[pix * 3 + 0] = cr[k];
      a.image[pix * 3 + 1] = cg[k];
      a.image[pix * 3 + 2] = cb[k];
      a.final_t[pix] = T[k];
      a.n_contrib[pix] = ncon[k];
    }
  }
  if (write_key) {
    // The tile's largest contributor count (pixels outside the image hold 0).
    int m = 0;
#pragma unroll
    for (int k = 0; k < PIX; ++k) m = max(m, ncon[k]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = max(m, __shfl_xor(m, o, 64));
    if (lane == 0) {
      a.tile_keys[tile] = uint32_t(min(m, 0xFFFF));
      a.tile_keys[a.num_tiles + tile] = uint32_t(checkpoint_count(start, m, list_len));
    }
  }
}

// kCompositeWaves waves per workgroup, one work item each (composite_item);
// workgroups are mapped onto XCDs so that each XCD takes one region of the
// plan (xcd_swizzle).  QUARTERS: the launch's items are quarters (every tile
// split); a whole-tile item is then composited as its four quarters in turn.
// Otherwise items are whole tiles; of a tile split into several items the
// first composites the whole tile and the others have no work.  Each kernel
// thus composites every pixel of any plan exactly once, with one instance of
// the walk (two would share one register allocation).
template <int TILE, bool ELLIPSOID, bool QUARTERS, bool CKPT, bool HITS>
__global__ __launch_bounds__(kCompositeWaves * 64) void composite_fwd_kernel(CompositeArgs a) {
  constexpr int NPIX = TILE * TILE;
  constexpr int PIX_TILE = NPIX >= 64 ? NPIX / 64 : 1;
  const int lane = threadIdx.x & 63;
  // Wave index held in a scalar register, so the item, tile and view indices
  // derived from it are scalar too.
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // The wave's current 64 entries, three float4 per entry (u, v, o, pa),
  // (pb, pc, r, g), (b, cut, -, -): written once per lane, then read as LDS
  // broadcasts per entry instead of ten v_readlane.
  __shared__ float4 chunk[kCompositeWaves][64][3];
  // The second batch of a two-batch step (checkpoint kernel only).
  __shared__ float4 chunk2[kCompositeWaves][CKPT ? 64 : 1][3];
  __shared__ int ck_slots[kCompositeWaves][CKPT ? kMaxCheckpoints : 1];  // a wave's records
  const int slot = xcd_swizzle(blockIdx.x, gridDim.x) * kCompositeWaves + wid;
  int tile, kind, index;
  if (!composite_item(a.items, a.num_items, a.num_tiles, a.split_all, slot, tile, kind, index))
    return;
  // Items that split a tile some other way (a backward plan's segments) are
  // composited whole by the tile's first item.
  if (kind != kItemTile && !(QUARTERS && kind == kItemQuarter) && index != 0) return;
  if constexpr (QUARTERS) {
    static_assert(PIX_TILE >= kCompositeWaves, "quarters of 64-pixel bands");
    constexpr int QPIX = PIX_TILE / kCompositeWaves;
    if (kind == kItemQuarter) {
      composite_tile<TILE, ELLIPSOID, QPIX, HITS>(a, chunk[wid], chunk2[wid], ck_slots[wid], lane,
                                                  tile, index * QPIX, false, false);
    } else {
      for (int q = 0; q < kCompositeWaves; ++q)
        composite_tile<TILE, ELLIPSOID, QPIX, HITS>(a, chunk[wid], chunk2[wid], ck_slots[wid],
                                                    lane, tile, q * QPIX, false, false);
    }
  } else {
    composite_tile<TILE, ELLIPSOID, PIX_TILE, HITS, CKPT>(a, chunk[wid], chunk2[wid],
                                                          ck_slots[wid], lane, tile, 0, CKPT, true);
  }
}

template <int TILE, bool QUARTERS, bool CKPT>
void launch_items(const CompositeArgs& a, bool ellipsoid, hipStream_t s) {
  const unsigned blocks = unsigned(
      a.items ? a.num_items / kCompositeWaves
              : (a.split_all ? a.num_tiles : ceil_div(a.num_tiles, kCompositeWaves)));
  if (ellipsoid)
    launch_timed(composite_fwd_kernel<TILE, true, QUARTERS, CKPT, false>, blocks, kCompositeWaves * 64, 0,
                 s, a);
  else if (a.hit_masks)
    launch_timed(composite_fwd_kernel<TILE, false, QUARTERS, CKPT, true>, blocks, kCompositeWaves * 64, 0,
                 s, a);
  else
    launch_timed(composite_fwd_kernel<TILE, false, QUARTERS, CKPT, false>, blocks, kCompositeWaves * 64, 0,
                 s, a);
}

// Checkpoint recording is a kernel of its own: the code for it costs the
// walk registers (73 VGPRs instead of 60 at tile 16, 6 waves per SIMD
// instead of 8), which only long lists repay.
template <int TILE>
void launch(const CompositeArgs& a, bool ellipsoid, hipStream_t s) {
  if constexpr (TILE >= 16) {
    if (a.split_all) return launch_items<TILE, true, false>(a, ellipsoid, s);
  }
  if constexpr (TILE <= 16) {
    if (a.ckpt_counter) return launch_items<TILE, false, true>(a, ellipsoid, s);
  }
  launch_items<TILE, false, false>(a, ellipsoid, s);
}

}  // namespace
}  // namespace gs

using namespace gs;

// Resets the pool counter and stamps the table with the walk's geometry
// (magic 0 when the walk records nothing into this buffer).
__global__ void checkpoint_clear_kernel(uint32_t* counter, uint32_t magic, uint32_t tile_size,
                                        uint32_t num_tiles, uint32_t table_len) {
  counter[0] = 0u;
  counter[1] = magic;
  counter[2] = tile_size;
  counter[3] = num_tiles;
  counter[4] = table_len;
}

extern "C" GS_API size_t gs_composite_checkpoint_bytes(gs_view view, int64_t num_intersections,
                                                       int64_t longest_list) {
  if (check_view(view, true) != GS_OK || num_intersections < 0) return 0;
  if (longest_list <= kCheckpointMinList) return 0;  // no walk would record one
  if (view.tile_size > 16) return 0;  // 16 pixels per lane leave no registers for them
  const Mosaic m = mosaic_of(view);
  if (dispatch_plan(m.num_tiles(), view.tile_size, view.active_tiles, false).split_all) return 0;
  return checkpoint_layout(nullptr, view.tile_size, num_intersections).bytes;
}

extern "C" GS_API size_t gs_composite_hit_mask_bytes(gs_view view, int64_t num_intersections) {
  if (check_view(view, true) != GS_OK || num_intersections < 0) return 0;
  const Mosaic m = mosaic_of(view);
  return size_t(hit_mask_words(num_intersections, m.num_tiles(), view.tile_size)) * 8;
}

extern "C" GS_API int gs_composite(const void* records, int64_t num_records,
                                   const int32_t* gaussian_ids, int64_t num_intersections,
                                   const int64_t* ranges, const int32_t* tile_order, gs_view view,
                                   float* image, float* final_transmittance,
                                   int32_t* n_contributors, void* checkpoints,
                                   size_t checkpoint_bytes, uint64_t* hit_masks,
                                   size_t hit_mask_bytes, uint32_t* tile_keys,
                                   size_t tile_keys_bytes, void* stream) {
  clear_error();
  GS_TRY(check_view(view, true));
  GS_REQUIRE(ranges && image && final_transmittance && n_contributors, GS_ERR_INVALID_ARGUMENT,
             "null pointer argument");
  GS_REQUIRE(num_records >= 0 && num_records <= (int64_t(1) << 31), GS_ERR_INVALID_ARGUMENT,
             "invalid record count %lld", (long long)num_records);
  GS_REQUIRE(num_records == 0 || records, GS_ERR_INVALID_ARGUMENT, "null records");
  GS_REQUIRE((reinterpret_cast<uintptr_t>(records) & 15u) == 0, GS_ERR_INVALID_ARGUMENT,
             "records must be 16-byte aligned");
  CompositeArgs a;
  a.records = static_cast<const GsRecord*>(records);
  a.max_id = uint32_t(num_records > 0 ? num_records - 1 : 0);
  a.ids = gaussian_ids;
  a.ranges = ranges;
  a.width = view.image_width;
  a.height = view.image_height;
  a.tile = view.tile_size;
  const Mosaic m = mosaic_of(view);
  a.tiles_w = m.tiles_w();
  a.num_tiles = m.num_tiles();
  a.view_tw = m.tw;
  a.view_th = m.th;
  a.cols = m.cols;
  a.views = m.views;
  a.threshold = view.opacity_threshold;
  a.t_active = float(1.0 - double(view.opacity_threshold));
  a.image = image;
  a.final_t = final_transmittance;
  a.n_contrib = n_contributors;
  const DispatchPlan plan = dispatch_plan(a.num_tiles, view.tile_size, view.active_tiles, false);
  a.items = tile_order;
  a.num_items = plan.items();
  a.split_all = plan.split_all;
  GS_REQUIRE(num_intersections >= 0, GS_ERR_INVALID_ARGUMENT, "negative intersection count");
  a.ckpt_counter = nullptr;
  a.ckpt_table = nullptr;
  a.ckpt_records = nullptr;
  a.ckpt_capacity = 0;
  a.hit_masks = hit_masks;
  a.hit_capacity = 0;
  GS_REQUIRE(!tile_keys || tile_keys_bytes >= size_t(a.num_tiles) * 2 * sizeof(uint32_t),
             GS_ERR_WORKSPACE, "tile key buffer too small (%zu bytes, need %zu)",
             tile_keys_bytes, size_t(a.num_tiles) * 2 * sizeof(uint32_t));
  // Keys come from whole-tile walks; with every tile split into quarters the
  // backward's plan computes them itself.
  a.tile_keys = plan.split_all ? nullptr : tile_keys;
  if (hit_masks) {
    GS_REQUIRE(view.rendering_mode == GS_MODE_GAUSSIAN, GS_ERR_UNSUPPORTED,
               "hit masks are recorded for Gaussian rendering only (its backward reads them)");
    const int64_t words = hit_mask_words(num_intersections, a.num_tiles, view.tile_size);
    GS_REQUIRE(hit_mask_bytes >= size_t(words) * 8, GS_ERR_WORKSPACE,
               "hit mask buffer too small (%zu bytes, need %zu)", hit_mask_bytes,
               size_t(words) * 8);
    GS_REQUIRE((reinterpret_cast<uintptr_t>(hit_masks) & 7u) == 0, GS_ERR_INVALID_ARGUMENT,
               "hit masks must be 8-byte aligned");
    a.hit_capacity = words;
  }
  hipStream_t s = as_stream(stream);
  if (checkpoints) {
    const CheckpointLayout c =
        checkpoint_layout(checkpoints, view.tile_size, num_intersections, checkpoint_bytes);
    GS_REQUIRE(checkpoint_bytes >= c.header_bytes, GS_ERR_WORKSPACE,
               "checkpoint buffer too small (%zu bytes, need at least %zu)", checkpoint_bytes,
               c.header_bytes);
    GS_REQUIRE((reinterpret_cast<uintptr_t>(checkpoints) & 255u) == 0, GS_ERR_INVALID_ARGUMENT,
               "checkpoint buffer must be 256-byte aligned");
    // The walk records checkpoints only in whole-tile waves of at most 16
    // pixels per lane; otherwise the stamp tells a backward that the table
    // holds nothing.
    const bool record = !plan.split_all && view.tile_size <= 16 && num_records > 0;
    if (record) {
      a.ckpt_counter = c.counter;
      a.ckpt_table = c.table;
      a.ckpt_records = c.records;
      a.ckpt_capacity = c.capacity;
    }
    checkpoint_clear_kernel<<<1, 1, 0, s>>>(c.counter, record ? kCheckpointMagic : 0u,
                                            uint32_t(view.tile_size), uint32_t(a.num_tiles),
                                            uint32_t(c.table_len));
    GS_TRY(check_launch("composite checkpoints"));
  }
  const bool ellipsoid = view.rendering_mode == GS_MODE_ELLIPSOID;
  switch (view.tile_size) {
    case 4: launch<4>(a, ellipsoid, s); break;
    case 8: launch<8>(a, ellipsoid, s); break;
    case 16: launch<16>(a, ellipsoid, s); break;
    default: launch<32>(a, ellipsoid, s); break;
  }
  return check_launch("composite");
}
