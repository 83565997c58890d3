// Backward compositing: one wave64 per work item (a whole tile, or a quarter
// of a heavy tile's pixel bands: the dispatch plan of tile_order.hip),
// back-to-front over the entries each pixel processed while active (positions
// < n_contributors).
//
// Exact gradient of the forward of composite_fwd.hip (the function
// torch.py:172-225 defines, differentiated as autograd would):
//   T_i    = T_{i+1} / (1 - alpha_i)            (T_{last+1} = final T)
//   dC/dc_i     = T_i alpha_i
//   dC/dalpha_i = T_i (c_i - S_i),  S_{i-1} = alpha_i c_i + (1 - alpha_i) S_i
// with zero gradient through the 1/255 cut, the active mask and, for the
// opacity/mean/conic, where o * G > 0.99 (clamp_max passes the gradient for
// inputs <= 0.99).  Only g . S (g = dL/dC of the pixel) is carried, as
// g . S_{i-1} = alpha_i (g . c_i) + (1 - alpha_i) g . S_i.
//
// Per Gaussian, each lane sums over its pixels (which share one column, so one
// dx) q = dL/dalpha * G, q dy, q dy^2 and g T alpha, folds them into the nine
// per-lane partial gradients
//   (u, v, inv00, inv01, inv11, r, g, b, opacity) += (-2 k (a Sx + b Sy),
//   -2 k (b Sx + c Sy), k Sxx, k Sxy, k Syy, Sr, Sg, Sb, Sq),  k = -o / 2,
// and the wave sums them with a transposing permlane/DPP reduction that leaves
// them in four rows of three registers; two fp32 atomic adds (four and five
// lanes) write them, once per (tile, Gaussian).  Replaces composite_bwd.py:47-204 and the
// index_add_ scatter of composite_bwd.py:268-273.
#include "common.h"
#include "raster_math.h"

namespace gs {
namespace {

struct CompositeBwdArgs {
  const float* pmean;
  const float* pinv;
  const float* pcolor;
  const float* popacity;
  uint32_t max_id;  // last valid Gaussian index: every gathered id is clamped to it
  const int32_t* ids;
  const int64_t* ranges;
  const int32_t* items;  // dispatch plan (gs_tile_order), or nullptr: tiles in index order
  int num_items;
  bool split_all;        // without a plan: every tile split into quarters
  const float* grad_image;
  const float* final_t;
  const int32_t* n_contrib;
  int width, height;       // per view
  int tiles_w, num_tiles;  // of the whole mosaic
  int view_tw, view_th, cols, views;  // tiles per view, mosaic layout (one view: cols = views = 1)
  float* grad;      // [N, 9]
  float* grad_abs;  // [N, 2]: sums of |per-pixel mean gradient| (ABS kernels only)
  // The forward's checkpoints (CheckpointLayout), or null table: none.  The
  // table is used only when the forward's stamp matches this view.
  const int32_t* ckpt_table;
  const float4* ckpt_records;
  int64_t ckpt_capacity;
  const uint32_t* ckpt_stamp;
  uint32_t ckpt_table_len;
  // The forward's hit masks (hit_mask_slot), read by the MASKS kernels.
  const uint64_t* hit_masks;
  int64_t hit_capacity;  // words
};

// One wave takes PIX pixels per lane of `tile`: the 64-pixel bands band0 ..
// band0 + PIX - 1 (all of them for a whole-tile item, a quarter for a quarter
// item), walking back from its own pixels' largest contributor count, and
// adds their share of every gradient.  A segment item (seg >= 0, all of the
// tile's bands) walks only the positions between two of the forward's
// checkpoints of the tile, [B_seg, B_seg+1) (B_0 = 0; the last segment runs
// to the largest contributor count), starting at B_seg+1 from that
// checkpoint's record: T there, and g.S = g . (colour composited after it) /
// T, the state the walk back from the end would reach there (the
// associative combine of back-to-front compositing, composite_bwd.py:24-36).
// Segments past the last recorded checkpoint (a full pool) have no work; the
// one at it runs to the end.
// The walk takes the list in the forward's batches of 64 entries (lane j:
// entry j of the batch), last batch first; each lane tests its entry's reach
// of every band's active pixels.  MASKS: only the entries the forward's masks
// mark (those that reached its active pixels) are gathered and tested.
template <int TILE, bool ABS, int PIX, bool MASKS>
__device__ __forceinline__ void composite_bwd_tile(const CompositeBwdArgs& a, float4 (*chunk)[3],
                                                   int lane, int tile, int band0, int seg) {
  constexpr int NPIX = TILE * TILE;
  constexpr int kBandRows = 64 / TILE > 0 ? 64 / TILE : 1;  // tile rows per band of 64 pixels

  // Mosaic tile -> view and the tile's pixel origin inside that view.
  const int tx = tile % a.tiles_w;
  const int ty = tile / a.tiles_w;
  const int vx = tx / a.view_tw, vy = ty / a.view_th;
  const int view = vy * a.cols + vx;
  if (view >= a.views) return;  // an empty slot of the mosaic's last row
  const int ox = (tx - vx * a.view_tw) * TILE, oy = (ty - vy * a.view_th) * TILE;
  const int64_t view_base = int64_t(view) * a.width * a.height;  // first pixel of the view
  const int64_t start = a.ranges[2 * tile];

  // The lane's pixels share one column (see column_terms).
  const float pxf = float(ox + lane % TILE);
  float pyf[PIX];
  float T[PIX], gr[PIX], gg[PIX], gb[PIX], gs_[PIX];
  int ncon[PIX];
  int max_n = 0;
#pragma unroll
  for (int k = 0; k < PIX; ++k) {
    const int q = lane + 64 * (band0 + k);
    const int px = ox + (q % TILE), py = oy + (q / TILE);
    const bool valid = q < NPIX && px < a.width && py < a.height;
    const int64_t pix = view_base + int64_t(py) * a.width + px;
    pyf[k] = float(py);
    T[k] = valid ? a.final_t[pix] : 1.0f;
    ncon[k] = valid ? a.n_contrib[pix] : 0;
    gr[k] = valid ? a.grad_image[pix * 3 + 0] : 0.0f;
    gg[k] = valid ? a.grad_image[pix * 3 + 1] : 0.0f;
    gb[k] = valid ? a.grad_image[pix * 3 + 2] : 0.0f;
    gs_[k] = 0.0f;
    max_n = max(max_n, ncon[k]);
  }
  // MASKS: each band's largest contributor count.  The forward's wave of a
  // band wrote the masks of every batch below it and may have stopped after
  // it, so later words of the band are never read.  The wave-wide maxima are
  // made scalar (readfirstlane), which keeps the walk's bounds in SGPRs.
  int band_hi[PIX];
  if constexpr (MASKS) {
    max_n = 0;
#pragma unroll
    for (int k = 0; k < PIX; ++k) {
      int m = ncon[k];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) m = max(m, __shfl_xor(m, o, 64));
      band_hi[k] = __builtin_amdgcn_readfirstlane(m);
      max_n = max(max_n, band_hi[k]);
    }
  } else {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) max_n = max(max_n, __shfl_xor(max_n, o, 64));
    max_n = __builtin_amdgcn_readfirstlane(max_n);
  }
  int lo = 0, hi = max_n;  // positions walked
  if (seg >= 0) {
    // Recorded checkpoints: a prefix of the tile's crossings (lane j reads
    // the table slot of crossing j + 1).
    const bool table =
        a.ckpt_table && a.ckpt_stamp[0] == kCheckpointMagic && a.ckpt_stamp[1] == uint32_t(TILE) &&
        a.ckpt_stamp[2] == uint32_t(a.num_tiles) && a.ckpt_stamp[3] == a.ckpt_table_len;
    const int m = table ? checkpoint_count(start, max_n, a.ranges[2 * tile + 1] - start) : 0;
    const int64_t first = checkpoint_first(start);
    const int slot = lane < m ? a.ckpt_table[(first + int64_t(lane) * kCheckpointEntries) /
                                             kCheckpointEntries]
                              : -1;
    // A slot outside the pool (never written by this forward) counts as missing.
    const uint64_t missing = __ballot(lane < m && (slot < 0 || int64_t(slot) >= a.ckpt_capacity));
    const int w = missing ? __builtin_ctzll(missing) : m;
    if (seg > w) return;
    lo = seg == 0 ? 0 : checkpoint_batch(start, seg);
    if (seg < w) {
      hi = checkpoint_batch(start, seg + 1);
      const float4* rec =
          a.ckpt_records + int64_t(__builtin_amdgcn_readlane(slot, seg)) * (PIX * 64);
#pragma unroll
      for (int p = 0; p < PIX; ++p) {
        const float4 v = rec[lane + 64 * (band0 + p)];
        T[p] = v.x;
        const float dot = gr[p] * v.y + gg[p] * v.z + gb[p] * v.w;
        gs_[p] = v.x > 0.0f ? dot / v.x : 0.0f;
      }
    }
    if (lo >= hi) return;
  }

  // Gradient fields written by this lane's two atomics: lane 16 r writes the
  // row-r fields of t0 and t1 of the nine-way sum, lane 1 the opacity total t2.
  const int field = sum9_field(lane >> 4);
  const bool row_writer = (lane & 15) == 0;
  const bool second_writer = row_writer || lane == 1;
  const int second_field = row_writer ? 4 + field : 8;

  // Each batch's ids are requested one batch ahead, once the current batch
  // is in LDS, so a batch waits on one dependent load (the gather), not two.
  constexpr int kBands = NPIX >= 64 ? NPIX / 64 : 1;  // the tile's 64-pixel bands
  const int64_t b_lo = lo >> 6;                   // lo is a multiple of 64
  const int64_t b_end = (int64_t(hi) + 63) >> 6;  // batches [b_lo, b_end)
  uint32_t next_id = b_end > b_lo && (b_end - 1) * 64 + lane < hi
                         ? uint32_t(a.ids[start + (b_end - 1) * 64 + lane])
                         : 0u;
  // MASKS: the OR of batch bt's masks of the wave's bands (wave-uniform),
  // requested one batch ahead.  The masks do not change during the launch:
  // read through the constant address space, the uniform reads are scalar
  // loads.
  using ConstMasks = const __attribute__((address_space(4))) uint64_t*;
  const ConstMasks masks = (ConstMasks)a.hit_masks;
  uint64_t next_walk = ~uint64_t(0);
  auto load_masks = [&](int64_t bt) {
    const int64_t w0 = hit_mask_slot(start, tile, bt) * kBands + band0;
    next_walk = 0;
#pragma unroll
    for (int k = 0; k < PIX; ++k)
      next_walk |=
          bt >= b_lo && bt * 64 < band_hi[k] && w0 + k < a.hit_capacity ? masks[w0 + k] : 0;
  };
  if constexpr (MASKS) load_masks(b_end - 1);
  for (int64_t bt = b_end - 1; bt >= b_lo; --bt) {
    const int pos0 = int(bt * 64);  // list position of lane 0's entry
    const bool valid = pos0 + lane < hi;
    const uint64_t walk = next_walk;  // MASKS: the entries to gather
    // Each band's overlap test takes the rectangle of its pixels active at
    // some position of the batch (ncon > pos0); a band with none is skipped.
    float bx0[PIX], bx1[PIX], by0[PIX], by1[PIX];
    uint32_t live_bands = 0;
#pragma unroll
    for (int k = 0; k < PIX; ++k) {
      const uint64_t m = __ballot(pos0 < ncon[k]);
      bx0[k] = bx1[k] = by0[k] = by1[k] = 0.0f;
      if (m) {
        uint32_t c;
        int r0, r1;
        band_span<TILE>(m, c, r0, r1);
        bx0[k] = float(ox + __builtin_ctz(c));
        bx1[k] = float(ox + 31 - __builtin_clz(c));
        by0[k] = float(oy + (band0 + k) * kBandRows + r0);
        by1[k] = float(oy + (band0 + k) * kBandRows + r1);
        live_bands |= 1u << k;
      }
    }
    LaneSplat mine;
    int gid = 0;
    uint32_t bands = 0;  // bit k: the Gaussian can reach an active pixel of band k
    if (valid && live_bands && ((walk >> lane) & 1u)) {
      gid = int(min(next_id, a.max_id));
      const GsRecord rec = load_projected(a.pmean, a.pinv, a.pcolor, a.popacity, gid);
#pragma unroll
      for (int k = 0; k < PIX; ++k) {
        if (((live_bands >> k) & 1u) && touches_rect(rec, bx0[k], bx1[k], by0[k], by1[k]))
          bands |= 1u << k;
      }
      mine = lane_splat(rec);
    }
    chunk[lane][0] = make_float4(mine.u, mine.v, mine.o, mine.pa);
    chunk[lane][1] = make_float4(mine.pb, mine.pc, mine.r, mine.g);
    chunk[lane][2] = make_float4(mine.b, mine.oa, mine.ob, mine.oc);
    next_id = bt - 1 >= b_lo ? uint32_t(a.ids[start + (bt - 1) * 64 + lane]) : 0u;
    if constexpr (MASKS) load_masks(bt - 1);
    uint64_t mask = __ballot(bands != 0);
    while (mask) {
      const int j = 63 - __builtin_clzll(mask);  // back to front
      mask &= ~(uint64_t(1) << j);
      const uint32_t band_mask = uint32_t(__builtin_amdgcn_readlane(int(bands), j));
      const float4 f0 = chunk[j][0], f1 = chunk[j][1], f2 = chunk[j][2];
      Splat s;
      s.u = f0.x;
      s.v = f0.y;
      s.o = f0.z;
      s.pa = f0.w;
      s.pb = f1.x;
      s.pc = f1.y;
      s.cut = 0.0f;  // Gaussian mode only
      s.r = f1.z;
      s.g = f1.w;
      s.bl = f2.x;
      const int pos = pos0 + j;
      const ColumnTerms c = column_terms(s, pxf);
      // Per-lane sums over the lane's pixels; -0 is the identity of +, so the
      // first term needs no add.
      float s0 = -0.0f, s1 = -0.0f, s2 = -0.0f;  // sum q, q dy, q dy^2
      float sr = -0.0f, sg = -0.0f, sb = -0.0f;
      float ax = -0.0f, ay = -0.0f;  // ABS: sum |q (oa dx + ob dy)|, |q (ob dx + oc dy)|
      const float oa = f2.y, ob = f2.z, oc = f2.w;
      const float oadx = oa * c.dx, obdx = ob * c.dx;
      bool touched = false;
      // Branch-free: an entry a pixel did not process while active, or whose
      // alpha is cut to 0, runs with alpha = 0, which leaves T, g.S and every
      // sum unchanged.
#pragma unroll
      for (int k = 0; k < PIX; ++k) {
        // A band of 64 pixels that the Gaussian cannot reach, or none of
        // which processed this entry, is skipped.
        if (!((band_mask >> k) & 1u) || __ballot(pos < ncon[k]) == 0) continue;
        const float dy = pyf[k] - s.v;
        float prob;
        const float raw = raw_alpha<false>(s, c, dy, prob);
        const float clamped = fminf(raw, kMaxAlpha);
        const bool hit = pos < ncon[k] && clamped >= kMinAlpha;
        const float alpha = hit ? clamped : 0.0f;
        touched |= hit;
        // T before the entry = T after it / (1 - alpha), with 1 / (1 - alpha)
        // formed as 1 + alpha / (1 - alpha): v_rcp_f32's error (up to an ulp,
        // of one sign) then enters scaled by alpha, so walking back through
        // thousands of small-alpha entries does not accumulate it (with the
        // plain reciprocal: ~2e-4 relative after 1600 entries).  alpha = 0
        // gives exactly 1.
        const float t_before = T[k] * fmaf(alpha, __builtin_amdgcn_rcpf(1.0f - alpha), 1.0f);
        const float w = t_before * alpha;
        sr += gr[k] * w;
        sg += gg[k] * w;
        sb += gb[k] * w;
        const float gc = gr[k] * s.r + gg[k] * s.g + gb[k] * s.bl;
        const float diff = gc - gs_[k];
        gs_[k] += alpha * diff;
        T[k] = t_before;
        // dL/dalpha * G where alpha is neither cut nor clamped (alpha == raw
        // holds exactly then, and never for a cut or clamped alpha with G > 0).
        const float q = alpha == raw ? t_before * diff * prob : 0.0f;
        const float qy = q * dy;
        s0 += q;
        s1 += qy;
        s2 += qy * dy;
        if constexpr (ABS) {
          ax += fabsf(q * fmaf(ob, dy, oadx));
          ay += fabsf(q * fmaf(oc, dy, obdx));
        }
      }
      if (__ballot(touched) == 0) continue;
      // d alpha / d(u, v, conic) folded per lane before the reduction
      // (k = -o/2, -2k = o):  u: o (a Sx + b Sy),  v: o (b Sx + c Sy),
      // inv00: k Sxx,  inv01: k Sxy,  inv11: k Syy,  Sx = dx s0, Sxx = dx^2 s0,
      // Sxy = dx s1, Sy = s1, Syy = s2.
      const float sx = c.dx * s0;
      const float kdx = (-0.5f * s.o) * c.dx;
      float v[9];
      v[0] = oa * sx + ob * s1;
      v[1] = ob * sx + oc * s1;
      v[2] = kdx * sx;
      v[3] = kdx * s1;
      v[4] = (-0.5f * s.o) * s2;
      v[5] = sr;
      v[6] = sg;
      v[7] = sb;
      v[8] = s0;
      float t0, t1, t2;
      wave_sum9(v, t0, t1, t2);
      float* dst = a.grad + int64_t(__builtin_amdgcn_readlane(gid, j)) * 9;
      if (row_writer) unsafeAtomicAdd(dst + field, t0);
      if (second_writer) unsafeAtomicAdd(dst + second_field, row_writer ? t1 : t2);
      if constexpr (ABS) {
        // Lanes 0-31 fold |du| terms, 32-63 |dv| terms; then every lane of
        // rows 0-1 holds the |du| total and of rows 2-3 the |dv| total.
        const float h = fold_halves(ax, ay);
        const float tabs = row_sum(fold_rows(h, h));
        if ((lane & 31) == 0)
          unsafeAtomicAdd(a.grad_abs + int64_t(__builtin_amdgcn_readlane(gid, j)) * 2 + (lane >> 5),
                          tabs);
      }
    }
  }
}

// kCompositeWaves waves per workgroup, one work item each (composite_item);
// workgroups are mapped onto XCDs so that each XCD takes one region of the
// plan (xcd_swizzle).  QUARTERS: the launch's items are quarters (every tile
// split); a whole-tile item is then composited as its four quarters in turn.
// Otherwise items are whole tiles; of a tile's four quarter items the first
// composites the whole tile and the others have no work.  Each kernel thus
// composites every pixel of any plan exactly once, with one instance of the
// walk (two would share one register allocation).
template <int TILE, bool ABS, bool QUARTERS, bool MASKS>
__global__ __launch_bounds__(kCompositeWaves * 64) void composite_bwd_kernel(CompositeBwdArgs a) {
  constexpr int NPIX = TILE * TILE;
  constexpr int PIX_TILE = NPIX >= 64 ? NPIX / 64 : 1;
  const int lane = threadIdx.x & 63;
  // Wave index held in a scalar register, so the item, tile and view indices
  // derived from it are scalar too.
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // The wave's current 64 entries, three float4 per entry (u, v, o, pa),
  // (pb, pc, r, g), (b, oa, ob, oc): written once per lane, then read as LDS
  // broadcasts per entry instead of twelve v_readlane.
  __shared__ float4 chunk[kCompositeWaves][64][3];
  const int slot = xcd_swizzle(blockIdx.x, gridDim.x) * kCompositeWaves + wid;
  int tile, kind, index;
  if (!composite_item(a.items, a.num_items, a.num_tiles, a.split_all, slot, tile, kind, index))
    return;
  if constexpr (QUARTERS) {
    static_assert(PIX_TILE >= kCompositeWaves, "quarters of 64-pixel bands");
    constexpr int QPIX = PIX_TILE / kCompositeWaves;
    if (kind == kItemQuarter) {
      composite_bwd_tile<TILE, ABS, QPIX, MASKS>(a, chunk[wid], lane, tile, index * QPIX, -1);
    } else if (kind == kItemTile || index == 0) {  // a segmented tile whole, by its first item
      for (int q = 0; q < kCompositeWaves; ++q)
        composite_bwd_tile<TILE, ABS, QPIX, MASKS>(a, chunk[wid], lane, tile, q * QPIX, -1);
    }
  } else {
    if (kind == kItemQuarter && index != 0) return;  // the tile whole, by its first quarter
    composite_bwd_tile<TILE, ABS, PIX_TILE, MASKS>(a, chunk[wid], lane, tile, 0,
                                                   kind == kItemSegment ? index : -1);
  }
}

template <int TILE, bool QUARTERS, bool MASKS>
void launch_masks(const CompositeBwdArgs& a, unsigned blocks, hipStream_t s) {
  if (a.grad_abs)
    launch_timed(composite_bwd_kernel<TILE, true, QUARTERS, MASKS>, blocks, kCompositeWaves * 64, 0, s, a);
  else
    launch_timed(composite_bwd_kernel<TILE, false, QUARTERS, MASKS>, blocks, kCompositeWaves * 64, 0, s, a);
}

template <int TILE, bool QUARTERS>
void launch_items(const CompositeBwdArgs& a, hipStream_t s) {
  const unsigned blocks = unsigned(
      a.items ? a.num_items / kCompositeWaves
              : (a.split_all ? a.num_tiles : ceil_div(a.num_tiles, kCompositeWaves)));
  if (a.hit_masks)
    launch_masks<TILE, QUARTERS, true>(a, blocks, s);
  else
    launch_masks<TILE, QUARTERS, false>(a, blocks, s);
}

template <int TILE>
void launch(const CompositeBwdArgs& a, hipStream_t s) {
  if constexpr (TILE >= 16) {
    if (a.split_all) return launch_items<TILE, true>(a, s);
  }
  launch_items<TILE, false>(a, s);
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" GS_API int gs_composite_bwd(const float* projected_mean,
                                       const float* inverse_covariance,
                                       const float* projected_color,
                                       const float* projected_opacity, int64_t n,
                                       const int32_t* gaussian_ids, const int64_t* ranges,
                                       const float* grad_image, const float* final_transmittance,
                                       const int32_t* n_contributors, const int32_t* tile_order,
                                       gs_view view, float* grad_projected, float* grad_absolute,
                                       const void* checkpoints, size_t checkpoint_bytes,
                                       int64_t num_intersections, const uint64_t* hit_masks,
                                       size_t hit_mask_bytes, void* stream) {
  clear_error();
  GS_TRY(check_view(view, true));
  GS_REQUIRE(view.rendering_mode == GS_MODE_GAUSSIAN, GS_ERR_UNSUPPORTED,
             "Backward gradients are only supported for Gaussian rendering.");
  GS_REQUIRE(ranges && grad_image && final_transmittance && n_contributors && grad_projected,
             GS_ERR_INVALID_ARGUMENT, "null pointer argument");
  GS_REQUIRE((reinterpret_cast<uintptr_t>(inverse_covariance) & 15u) == 0,
             GS_ERR_INVALID_ARGUMENT, "inverse_covariance must be 16-byte aligned");
  GS_REQUIRE(n >= 0 && n <= (int64_t(1) << 31), GS_ERR_INVALID_ARGUMENT,
             "invalid Gaussian count %lld", (long long)n);
  GS_REQUIRE(n == 0 || (projected_mean && inverse_covariance && projected_color &&
                        projected_opacity),
             GS_ERR_INVALID_ARGUMENT, "null pointer argument");
  CompositeBwdArgs a;
  a.max_id = uint32_t(n > 0 ? n - 1 : 0);
  a.pmean = projected_mean;
  a.pinv = inverse_covariance;
  a.pcolor = projected_color;
  a.popacity = projected_opacity;
  a.ids = gaussian_ids;
  a.ranges = ranges;
  a.grad_image = grad_image;
  a.final_t = final_transmittance;
  a.n_contrib = n_contributors;
  a.width = view.image_width;
  a.height = view.image_height;
  const Mosaic m = mosaic_of(view);
  a.tiles_w = m.tiles_w();
  a.num_tiles = m.num_tiles();
  a.view_tw = m.tw;
  a.view_th = m.th;
  a.cols = m.cols;
  a.views = m.views;
  a.grad = grad_projected;
  a.grad_abs = grad_absolute;
  const DispatchPlan plan = dispatch_plan(a.num_tiles, view.tile_size, view.active_tiles, true);
  a.items = tile_order;
  a.num_items = plan.items();
  a.split_all = plan.split_all;
  a.ckpt_table = nullptr;
  a.ckpt_records = nullptr;
  a.ckpt_capacity = 0;
  a.hit_masks = hit_masks;
  a.hit_capacity = 0;
  if (hit_masks) {
    GS_REQUIRE(num_intersections >= 0, GS_ERR_INVALID_ARGUMENT, "negative intersection count");
    const int64_t words = hit_mask_words(num_intersections, a.num_tiles, view.tile_size);
    GS_REQUIRE(hit_mask_bytes >= size_t(words) * 8, GS_ERR_WORKSPACE,
               "hit mask buffer too small (%zu bytes, need %zu)", hit_mask_bytes,
               size_t(words) * 8);
    GS_REQUIRE((reinterpret_cast<uintptr_t>(hit_masks) & 7u) == 0, GS_ERR_INVALID_ARGUMENT,
               "hit masks must be 8-byte aligned");
    a.hit_capacity = words;
  }
  a.ckpt_stamp = nullptr;
  a.ckpt_table_len = 0;
  // The forward records checkpoints under these conditions only
  // (composite_fwd.hip); its stamp is checked on the device as well.
  if (checkpoints && !plan.split_all && view.tile_size <= 16 && n > 0) {
    GS_REQUIRE(num_intersections >= 0, GS_ERR_INVALID_ARGUMENT, "negative intersection count");
    const CheckpointLayout c = checkpoint_layout(const_cast<void*>(checkpoints), view.tile_size,
                                                 num_intersections, checkpoint_bytes);
    GS_REQUIRE(checkpoint_bytes >= c.header_bytes, GS_ERR_WORKSPACE,
               "checkpoint buffer too small (%zu bytes, need at least %zu)", checkpoint_bytes,
               c.header_bytes);
    GS_REQUIRE((reinterpret_cast<uintptr_t>(checkpoints) & 255u) == 0, GS_ERR_INVALID_ARGUMENT,
               "checkpoint buffer must be 256-byte aligned");
    a.ckpt_table = c.table;
    a.ckpt_records = c.records;
    a.ckpt_capacity = c.capacity;
    a.ckpt_stamp = c.stamp;
    a.ckpt_table_len = uint32_t(c.table_len);
  }
  hipStream_t s = as_stream(stream);
  switch (view.tile_size) {
    case 4: launch<4>(a, s); break;
    case 8: launch<8>(a, s); break;
    case 16: launch<16>(a, s); break;
    default: launch<32>(a, s); break;
  }
  return check_launch("composite_bwd");
}
