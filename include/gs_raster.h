/*
 * gs_raster.h — C ABI of the MI355X (gfx950) differentiable Gaussian-splat
 * tile rasterizer.
 *
 * Every entry point takes raw device pointers, sizes as int64_t, scalars by
 * value and an explicit HIP stream (`void*` holding a hipStream_t; NULL is
 * the null stream).  The library never allocates, frees or synchronises:
 * the caller owns every buffer, including scratch space sized by the
 * matching *_workspace_bytes() query.  Functions return GS_OK (0) or a
 * gs_status code; the message for the calling thread is available from
 * gs_last_error().  All entry points are reentrant.
 *
 * Layouts (row-major, fp32 unless stated; these are the tensor layouts of
 * the reference's custom op, src/gaussian_splats/kernels/rasterize/
 * interface.py:17-49):
 *   mean[N,3], rotation[N,4] (w,x,y,z, unnormalised), scale[N,3] (log sigma),
 *   opacity[N,1] (logit), color[N,K,3] (coefficient-major, RGB innermost),
 *   camera_rotation[3,3] (world->camera), camera_translation[3] (both in
 *   host memory: the twelve values are passed to the kernels as arguments),
 *   projected_mean[N,3] (u, v, depth), inverse_covariance[N,2,2],
 *   projected_color[N,3], projected_opacity[N,1], bounds[N,2,2] int32
 *   (x_min, x_max, y_min, y_max in tiles, half-open), counts[N] int32,
 *   gaussian_ids[I] int32, ranges[T,2] int64 (half-open per tile),
 *   image[H,W,3], final_transmittance[H,W], n_contributors[H,W] int32,
 *   grad_projected[N,9] (u, v, inv00, inv01, inv11, r, g, b, opacity).
 * A "record" is the 48-byte packed per-Gaussian block the compositing
 * kernels gather: {u, v, opacity, depth}, {inv00, inv01, inv11, cut},
 * {r, g, b, 0}.
 *
 * Tiles: tiles_w = ceil(W / tile_size), tiles_h = ceil(H / tile_size);
 * pixels outside the image in the last tile row/column are masked.
 */
#ifndef GS_RASTER_H
#define GS_RASTER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GS_API __attribute__((visibility("default")))

#define GS_ABI_VERSION 17

typedef enum gs_status {
  GS_OK = 0,
  GS_ERR_INVALID_ARGUMENT = 1,
  GS_ERR_UNSUPPORTED = 2,
  GS_ERR_OVERFLOW = 3,
  GS_ERR_HIP = 4,
  GS_ERR_WORKSPACE = 5
} gs_status;

typedef enum gs_rendering_mode {
  GS_MODE_GAUSSIAN = 0,
  GS_MODE_ELLIPSOID = 1
} gs_rendering_mode;

/* Camera intrinsics, image/tile geometry and culling planes, passed by value.
 * Mirrors the scalar arguments of the reference op
 * (src/gaussian_splats/kernels/rasterize/interface.py:26-37). */
typedef struct gs_view {
  float fx, fy, cx, cy;
  int32_t image_width, image_height;
  int32_t tile_size;
  float near_plane, far_plane;
  int32_t rendering_mode;      /* gs_rendering_mode */
  float confidence;            /* ellipsoid mode only */
  float opacity_threshold;     /* compositing stops once 1 - T >= this */
  float covariance_epsilon;    /* 0.03 in the reference (camera.py:86) */
  /* Several views of one size composited in one launch (no counterpart in
   * the reference): their tile grids are laid side by side, mosaic_cols per
   * row, and tile t of the mosaic belongs to view (ty / tiles_h) *
   * mosaic_cols + tx / tiles_w.  Per-view buffers (image, transmittance,
   * contributors, image gradient) are [views, H, W, ...]; ranges cover the
   * mosaic's tiles.  0 or 1 in both fields: a single view. */
  int32_t views;
  int32_t mosaic_cols;
  /* Tiles with a non-empty list (totals[3] of gs_bin_tiles_plan), or 0 when
   * unknown.  The compositing calls split each tile's pixels over four waves
   * when fewer than 4096 tiles have work (few or skewed tiles would leave
   * SIMDs idle behind their longest tiles); results do not depend on it. */
  int32_t active_tiles;
} gs_view;

/* ABI version of the loaded library (GS_ABI_VERSION). No counterpart in the
 * reference (it has no compiled library). */
GS_API int gs_abi_version(void);

/* Message describing the last failure on the calling thread ("" if none). */
GS_API const char* gs_last_error(void);

/* Kernel timing for benchmarks.  No counterpart in the reference (its
 * benchmark times whole calls on the host); for callers that measure one
 * kernel's duration per launch.  gs_arm_launch_events arms two hipEvent_t
 * (created beforehand; either may be null) for the calling thread's next
 * timed kernel: the main kernel of gs_project_and_count, gs_project_views,
 * gs_project_bwd, gs_project_bwd_views, gs_composite, gs_composite_bwd,
 * gs_ply_pack or gs_ply_unpack (the first one launched, for calls that
 * launch several).
 * That launch carries the events (hipExtLaunchKernel), so they take the
 * kernel's own start and end timestamps; hipEventElapsedTime of the pair is
 * its duration.  gs_disarm_launch_events disarms them and returns 1 if a
 * launch took them since they were armed, 0 if none did (the call failed
 * before its kernel, or had nothing to launch). */
GS_API int gs_arm_launch_events(void* start_event, void* stop_event);
GS_API int gs_disarm_launch_events(void);

/* Device-side check failures.  The binning and sort kernels validate what
 * they cannot check on the host (sizes passed between calls against the
 * plan's device totals, the bounded spin of their look-back waits, owner
 * windows) and, on a failure, leave their outputs incomplete and OR one of
 * these bits into a sticky word kept per GPU.  No counterpart in the
 * reference (its torch.sort and Triton kernels have no device-side checks). */
#define GS_DEVICE_SPIN_LIMIT 1u       /* a look-back wait hit its spin limit */
#define GS_DEVICE_WINDOW_OVERFLOW 2u  /* a workgroup's owner window exceeded its tile */
#define GS_DEVICE_SIZE_MISMATCH 4u    /* sizes passed by the host differ from the plan's */

/* Reads the sticky word of the stream's GPU into *flags after the work
 * enqueued on `stream` so far has completed (this call synchronises the
 * stream), and clears it when `clear` != 0.  gs_bin_tiles_plan also copies
 * the word (as of its copy of the totals) to host_totals[4].  That copy is
 * the only read without a synchronisation of its own: it precedes the
 * call's sort and the following gs_bin_tiles_emit, so a failure inside them
 * is reported by the next gs_bin_tiles_plan (or by this call), one binning
 * later.  The word is sticky, so no failure goes unreported. */
GS_API int gs_device_errors(uint32_t* flags, int32_t clear, void* stream);

/* Projection, SH colour, tile rectangle and culled count for N Gaussians.
 * Replaces project_and_count (src/gaussian_splats/kernels/rasterize/
 * project.py:256-345) with the camera semantics of splats/camera.py:81-124
 * and splats/utils.py:8-75.  num_sh in {1, 4, 9, 16} (SH degree <= 3).
 * `records` (N x 48 B) and `depth_keys` (N x u32: depth bits for counted
 * Gaussians, 0xFFFFFFFF otherwise) are optional (NULL = not written), and so
 * is `tile_rects` (N x u32, no counterpart in the reference: each counted
 * Gaussian's tile rectangle packed as x0 | (x1 - x0 - 1) << 8 | y0 << 16 |
 * (y1 - y0 - 1) << 24, 0xFFFFFFFF for the others; tile grids of at most
 * 256 x 256, else GS_ERR_UNSUPPORTED), the input of gs_bin_tiles_plan.
 * With tile_rects, `bounds` may be NULL (not written). */
GS_API int gs_project_and_count(
    const float* mean, const float* rotation, const float* scale,
    const float* opacity, const float* color, int64_t n, int32_t num_sh,
    const float* camera_rotation, const float* camera_translation,
    gs_view view,
    float* projected_mean, float* inverse_covariance, float* projected_color,
    float* projected_opacity, int32_t* bounds, int32_t* counts,
    void* records, uint32_t* depth_keys, uint32_t* tile_rects, void* stream);

/* Multi-view projection (no counterpart in the reference, which renders one
 * camera per call): gs_project_and_count for the V = max(view.views, 1)
 * cameras of a mosaic sharing the image size, tile size and culling planes of
 * `view`, each Gaussian's parameters read once per launch of up to 16
 * cameras.  Host arrays: camera_rotations [V, 9], camera_translations [V, 3],
 * intrinsics [V, 4] = (fx, fy, cx, cy) per camera, or NULL for view's.
 * Outputs are [V, N, ...] (view v's at Gaussian v * N).  bounds and
 * tile_rects are in the mosaic's tile grid (each view's rectangle shifted to
 * its tile origin, see gs_view.views), so binning V * N Gaussians over the
 * mosaic's tiles lists every view's tiles in one pass. */
GS_API int gs_project_views(
    const float* mean, const float* rotation, const float* scale,
    const float* opacity, const float* color, int64_t n, int32_t num_sh,
    const float* camera_rotations, const float* camera_translations,
    const float* intrinsics, gs_view view,
    float* projected_mean, float* inverse_covariance, float* projected_color,
    float* projected_opacity, int32_t* bounds, int32_t* counts,
    void* records, uint32_t* depth_keys, uint32_t* tile_rects, void* stream);

/* Packs the per-Gaussian compositing record from the op's projected outputs
 * (used when compositing is called stage-wise, as composite.py:110 is).
 * `cut` is derived from opacity and the rendering mode. No counterpart in the
 * reference (its compositor gathers the four arrays field by field,
 * composite.py:61-91). */
GS_API int gs_pack_records(
    const float* projected_mean, const float* inverse_covariance,
    const float* projected_color, const float* projected_opacity, int64_t n,
    gs_view view, void* records, void* stream);

/* Scratch for gs_emit_intersections / gs_bin_gaussians. */
GS_API size_t gs_scan_workspace_bytes(int64_t n);

/* Exclusive scan of counts in Gaussian order: offsets[0..n] (offsets[n] is the
 * intersection total, read back by the caller).  First half of
 * emit_intersections (intersections.py:51-52). */
GS_API int gs_scan_counts(
    const int32_t* counts, int64_t n, int64_t* offsets,
    void* workspace, size_t workspace_bytes, void* stream);

/* Emits reference-format keys (tile_id << 32 | depth bits) and Gaussian ids
 * in Gaussian-major order at the scanned offsets (total = offsets[n]).  Second
 * half of emit_intersections (intersections.py:10-41,65-73).  depths has
 * element stride depth_stride (3 for projected_mean[:, 2]). */
GS_API int gs_emit_intersections(
    const int32_t* bounds, const float* depths, int64_t depth_stride,
    const int64_t* offsets, int64_t n, int64_t total, int32_t tiles_w,
    int64_t* keys, int32_t* gaussian_ids, void* stream);

/* Scratch for gs_sort_intersections / gs_sort_tiles. */
GS_API size_t gs_sort_workspace_bytes(int64_t total, int32_t num_tiles);

/* Stable sort of reference-format 64-bit keys with their Gaussian ids
 * (ties keep emission order, i.e. ascending Gaussian id) and per-tile
 * half-open ranges.  Replaces sort_intersections (intersections.py:77-88).
 * keys/gaussian_ids are consumed (used as ping-pong buffers). */
GS_API int gs_sort_intersections(
    int64_t* keys, int32_t* gaussian_ids, int64_t total, int32_t num_tiles,
    int32_t* sorted_ids, int64_t* ranges,
    void* workspace, size_t workspace_bytes, void* stream);

/* Fused binning used by the op: orders counted Gaussians by (depth bits,
 * index), scans their counts in that order (offsets[0..n], offsets[n] =
 * total), so that emitting in that order and stably sorting by tile yields
 * exactly the order of the stable (tile, depth) key sort.  depth_keys (from
 * gs_project_and_count) is consumed as sort scratch.  Replaces the scan of
 * intersections.py:51-52. */
GS_API size_t gs_bin_workspace_bytes(int64_t n);
GS_API int gs_bin_gaussians(
    uint32_t* depth_keys, const int32_t* counts, int64_t n,
    int32_t* order, int64_t* offsets,
    void* workspace, size_t workspace_bytes, void* stream);

/* Emits 32-bit tile keys and Gaussian ids in depth order (order/offsets from
 * gs_bin_gaussians; total = offsets[n]).  Replaces the emit of
 * intersections.py:10-41. */
GS_API int gs_emit_tiles(
    const int32_t* bounds, const int32_t* order, const int64_t* offsets,
    int64_t n, int64_t total, int32_t tiles_w, uint32_t* tile_keys,
    int32_t* gaussian_ids, void* stream);

/* Stable LSD radix sort of (tile key, id) over ceil(log2 num_tiles) bits and
 * tile ranges; tile_keys/gaussian_ids are consumed.  Replaces
 * sort_intersections (intersections.py:77-88) for the fused path. */
GS_API int gs_sort_tiles(
    uint32_t* tile_keys, int32_t* gaussian_ids, int64_t total,
    int32_t num_tiles, int32_t* sorted_ids, int64_t* ranges,
    void* workspace, size_t workspace_bytes, void* stream);

/* Row-bucketed binning, used by the op when the tile grid is at most
 * 256 x 256 (otherwise GS_ERR_UNSUPPORTED) and n is below 2^26 (otherwise
 * GS_ERR_OVERFLOW); use the three calls above beyond either.  Same
 * sorted ids and ranges as gs_bin_gaussians + gs_emit_tiles + gs_sort_tiles,
 * i.e. the stable (tile, depth bits, index) order of intersections.py:10-88,
 * with the tile-row and tile-column buckets filled directly from the tile
 * rectangles (no intersection keys are materialised or sorted).
 *
 * gs_bin_tiles_plan: depth order, per-tile counts and `ranges` [T, 2] (final),
 * and device `totals` = {intersections, row-list entries, pass-B workgroups,
 * tiles with a non-empty list | the longest list << 32 (capped at 2^31 - 1)},
 * which size the ids and shape the compositing calls.  With `host_totals`
 * (5 x int64, pinned host memory for an asynchronous copy) the call returns
 * once the four totals have been copied there, and the low 32 bits of
 * host_totals[4] hold the device's sticky check-failure word (see
 * gs_device_errors) as of that copy: non-zero means an earlier binning or
 * sort call on this GPU left incomplete output.  The tables are built on a
 * side stream, so the host waits for them while the depth sort still runs on
 * `stream`; `stream` itself is then not made to wait for the side stream
 * (work enqueued on it after the call follows the side stream's), without
 * `host_totals` it is.  `plan` (plan_bytes from
 * gs_bin_tiles_plan_bytes) must stay alive until gs_bin_tiles_emit, which
 * takes the totals (device pointer and the values read from it) and writes
 * `sorted_ids` [totals[0]].  depth_keys and tile_rects are
 * gs_project_and_count's (depth_keys: ~0u for Gaussians without
 * intersections; consumed).  Together they replace intersections.py:44-88
 * for the op.  key_bits in [1, 32]: with 32 the depth order is that of the
 * keys' 32 bits (four sort passes); below 32 it is that of min(key -
 * key_base, 2^key_bits - 1) (keys below key_base or at least key_base +
 * 2^key_bits - 1 sort last, in index order), in ceil(key_bits / 8) passes
 * of near-equal width.  The op passes key_base = the bits of its float near
 * plane and key_bits = the bit length of bits(far) - bits(near): every
 * counted Gaussian's depth lies strictly between the planes, so the order is
 * the same (near 0.2, far 100: 27 bits, passes of 7, 7, 7 and 6 bits).
 * `clear` (optional, 16-byte aligned, clear_bytes a multiple of 4; no
 * counterpart in the reference) is zeroed on the side stream beside
 * the depth sort, before the totals are copied: the op passes the backward's
 * [N, 9] gradient accumulator, so no fill runs on `stream`. */
GS_API size_t gs_bin_tiles_plan_bytes(int64_t n, int32_t tiles_w, int32_t tiles_h);
GS_API int gs_bin_tiles_plan(
    uint32_t* depth_keys, const uint32_t* tile_rects, int64_t n, uint32_t key_base,
    int32_t key_bits, int32_t tiles_w, int32_t tiles_h, int64_t* ranges, int64_t* totals,
    int64_t* host_totals, void* plan, size_t plan_bytes, void* clear, size_t clear_bytes,
    void* stream);
/* tile_rects (the packing of gs_project_and_count) from bounds [N, 2, 2] and
 * counts, for callers holding those instead; no counterpart in the
 * reference. */
GS_API int gs_pack_tile_rects(
    const int32_t* bounds, const int32_t* counts, int64_t n, int32_t tiles_w, int32_t tiles_h,
    uint32_t* tile_rects, void* stream);
GS_API size_t gs_bin_tiles_emit_bytes(int64_t n, int64_t total, int64_t row_entries,
                                      int64_t blocks, int32_t tiles_w, int32_t tiles_h);
GS_API int gs_bin_tiles_emit(
    int64_t n, int32_t tiles_w, int32_t tiles_h,
    const int64_t* totals, int64_t total, int64_t row_entries, int64_t blocks,
    void* plan, size_t plan_bytes, const int64_t* ranges, int32_t* sorted_ids,
    void* workspace, size_t workspace_bytes, void* stream);

/* Dispatch plan of the compositing kernels (no counterpart in the reference,
 * whose launches take tiles in index order): writes
 * gs_tile_order_items(view, n_contributors != NULL) int32 work items to
 * tile_order.  Each item is one wave's work, tile << 7 | code: 0 the whole
 * tile; 0x20 | q quarter q of the tile's 64-pixel bands (tiles of 16 and 32
 * pixels when fewer than 4096 tiles have work: every tile split, a tile's
 * quarters in one workgroup's four slots); 0x40 | s segment s of the entries
 * the tile's pixels walk back, cut at the forward's checkpoints (see
 * gs_composite; backward plans given both ranges and n_contributors, the
 * heaviest tiles first while the region's spare slots last); -1 is an unused
 * slot.  The plan keeps each XCD's region of tiles and starts the tiles with
 * the most expected work first.  The work estimate is the list length from
 * ranges (a plan for gs_composite), or the largest contributor count of the
 * tile's pixels (a plan for gs_composite_bwd).  The compositing call takes
 * the plan made for it with the same view (tile size, mosaic and
 * active_tiles); its results do not depend on it.  The workspace holds two
 * words per tile: each tile's key, then its checkpoint crossings.  With
 * keys_ready (a backward plan), the workspace was passed as gs_composite's
 * tile_keys for the forward that produced n_contributors with this view, and
 * the keys it wrote are used instead of being recomputed (when that forward
 * split every tile into quarters it wrote none, and they are recomputed). */
GS_API size_t gs_tile_order_workspace_bytes(int32_t num_tiles);
GS_API int64_t gs_tile_order_items(gs_view view, int32_t by_contributors); /* -1: bad view */
GS_API int gs_tile_order(
    const int64_t* ranges, const int32_t* n_contributors, gs_view view,
    int32_t* tile_order, void* workspace, size_t workspace_bytes, int32_t keys_ready,
    void* stream);

/* gs_tile_order without a workspace argument (no counterpart in the
 * reference): for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc).  The tile
 * keys live in a static device array of the library, one per GPU, sized for
 * at most GS_TILE_ORDER_NOALLOC_MAX_TILES tiles (2 MiB); larger views are
 * rejected with GS_ERR_WORKSPACE.  Allocates nothing.  Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (different streams
 * or host threads) race and must be serialised by the caller. */
#define GS_TILE_ORDER_NOALLOC_MAX_TILES (1 << 18)
GS_API int gs_tile_order_noalloc(
    const int64_t* ranges, const int32_t* n_contributors, gs_view view,
    int32_t* tile_order, void* stream);

/* Front-to-back compositing per tile.  Replaces composite
 * (src/gaussian_splats/kernels/rasterize/composite.py:25-162) with the
 * pixel semantics of torch.py:172-225.  tile_size in {4, 8, 16, 32}.
 * `records` holds num_records records; gaussian_ids holds num_intersections
 * ids, clamped to [0, num_records), so incomplete lists (see
 * gs_device_errors) never read outside it.  tile_order: the dispatch plan of
 * gs_tile_order from ranges for this view, or NULL for tiles in index order
 * (split into quarters when fewer than 4096 tiles have work); it does not
 * change the results.
 * checkpoints (optional, gs_composite_checkpoint_bytes(view,
 * num_intersections) bytes, 256-byte aligned; no counterpart in the
 * reference): whenever a tile's walk starts a batch of 64 entries holding an
 * intersection index that is a multiple of 1024 (at least 64 past the tile's
 * first) of a list longer than 8192 entries, it records per pixel the
 * transmittance and the colour composited after that point (at most 63 per
 * tile, from a pool of at most 128 MiB), which gs_composite_bwd uses to walk
 * long lists back in segments at once.  The image is then the sum of the
 * colour before and after each record.  A smaller buffer is accepted down to
 * its header (counter, stamp and table): it holds as many records as fit,
 * and the crossings past them are marked missing, which the backward walks
 * without a record.  The forward stamps the buffer with its geometry (tile
 * size, tiles, table length), or clears the stamp when its walk records
 * nothing (tiles split into quarters, tile 32, no records); the backward
 * uses the table only when the stamp matches its own view.  The query returns 0 (no buffer
 * needed) when longest_list, the longest list (totals[3] >> 32 of
 * gs_bin_tiles_plan), is not above 8192, and for tiles of 32 pixels (whose
 * walk holds 16 pixels per lane, leaving no registers for the records). */
GS_API size_t gs_composite_checkpoint_bytes(gs_view view, int64_t num_intersections,
                                            int64_t longest_list);
/* hit_masks (optional, gs_composite_hit_mask_bytes(view, num_intersections)
 * bytes, 8-byte aligned; no counterpart in the reference): for every batch of
 * 64 entries of a tile's list that the walk processes, one 64-bit mask per
 * 64-pixel band of the tile, bit j set when entry j passed the walk's overlap
 * test, i.e. can reach alpha >= 1/255 inside the rectangle spanned by the
 * pixels still active at the batch's first entry.  gs_composite_bwd, given
 * the same buffer, gathers only the entries so marked (every entry that
 * contributes to a pixel is), instead of every entry of its walk.  The slots
 * assume the tiles' lists follow each other in tile order, as the binning
 * writes them; batches the walk does not reach are not written.  Gaussian
 * rendering only (GS_ERR_UNSUPPORTED otherwise).
 * tile_keys (optional, gs_tile_order_workspace_bytes(tiles) bytes; no
 * counterpart in the reference): a workspace for the backward's
 * gs_tile_order, filled as each tile's walk ends with its key (the largest
 * contributor count of its pixels, capped at 2^16 - 1) and its checkpoint
 * crossings, so that plan (keys_ready) does not read n_contributors again.
 * Not written when every tile is split into quarters. */
GS_API size_t gs_composite_hit_mask_bytes(gs_view view, int64_t num_intersections);
GS_API int gs_composite(
    const void* records, int64_t num_records, const int32_t* gaussian_ids,
    int64_t num_intersections, const int64_t* ranges, const int32_t* tile_order, gs_view view,
    float* image, float* final_transmittance, int32_t* n_contributors, void* checkpoints,
    size_t checkpoint_bytes, uint64_t* hit_masks, size_t hit_mask_bytes, uint32_t* tile_keys,
    size_t tile_keys_bytes, void* stream);

/* Back-to-front compositing gradient, accumulated with atomics into
 * grad_projected[N,9] (zeroed by the caller), from the op's projected outputs
 * of n Gaussians (list ids clamped to [0, n), as in gs_composite).
 * grad_absolute (optional, [N,2], zeroed by the caller) receives the sums of
 * the absolute per-pixel terms of the mean gradient, as composite_bwd.py's
 * return_absolute output (composite_bwd.py:180-185,194-195,272-277).
 * Replaces composite_bwd (composite_bwd.py:47-277) with the exact gradient of
 * the forward.  tile_order: the plan of gs_tile_order from n_contributors
 * (and ranges, for segments) for this view, or NULL (tiles in index order).
 * checkpoints: the buffer gs_composite filled for the same lists (or NULL):
 * a segment item starts its walk back at a checkpoint, with the
 * transmittance recorded there and g.S = g . (colour after it) / T, the
 * state the walk from the end would reach (the associative combine of
 * composite_bwd.py:24-36), so a long walk runs on many waves at once.  It is
 * read only where gs_composite records (whole tiles of at most 16 pixels, n
 * > 0) and only when its stamp matches this view; the stamp cannot tell two
 * walks of one geometry apart, so it must be the buffer of the forward over
 * these same lists.
 * hit_masks: the buffer gs_composite filled for the same lists and view (or
 * NULL: every entry of the walk is gathered and tested). */
GS_API int gs_composite_bwd(
    const float* projected_mean, const float* inverse_covariance,
    const float* projected_color, const float* projected_opacity, int64_t n,
    const int32_t* gaussian_ids, const int64_t* ranges,
    const float* grad_image, const float* final_transmittance,
    const int32_t* n_contributors, const int32_t* tile_order, gs_view view,
    float* grad_projected, float* grad_absolute, const void* checkpoints,
    size_t checkpoint_bytes, int64_t num_intersections, const uint64_t* hit_masks,
    size_t hit_mask_bytes, void* stream);

/* Chain rule from grad_projected to the parameters.  Replaces project_bwd
 * (src/gaussian_splats/kernels/rasterize/project_bwd.py:8-381); gradients are
 * zero for Gaussians with count == 0 (project_bwd.py:32,324-334).
 * inverse_covariance (the forward's output) is not read and may be null: the
 * covariance chain is recomputed from the parameters in double precision,
 * because for nearly degenerate 2-D covariances its gradient is far smaller
 * than the float32 products that would form it. */
GS_API int gs_project_bwd(
    const float* mean, const float* rotation, const float* scale,
    const float* opacity, const float* color, int64_t n, int32_t num_sh,
    const float* camera_rotation, const float* camera_translation,
    gs_view view, const float* inverse_covariance,
    const float* grad_projected, const int32_t* counts,
    float* grad_mean, float* grad_rotation, float* grad_scale,
    float* grad_opacity, float* grad_color, void* stream);

/* Multi-view projection backward (no counterpart in the reference): the
 * gradients gs_project_bwd gives for each of the V = max(view.views, 1)
 * cameras of gs_project_views, summed per Gaussian in registers and written
 * once (per 16 cameras).  inverse_covariance, grad_projected and counts are
 * [V, N, ...]; the camera arrays are those of gs_project_views. */
GS_API int gs_project_bwd_views(
    const float* mean, const float* rotation, const float* scale,
    const float* opacity, const float* color, int64_t n, int32_t num_sh,
    const float* camera_rotations, const float* camera_translations,
    const float* intrinsics, gs_view view, const float* inverse_covariance,
    const float* grad_projected, const int32_t* counts,
    float* grad_mean, float* grad_rotation, float* grad_scale,
    float* grad_opacity, float* grad_color, void* stream);

/* Photometric L1 loss of the training step that consumes the image
 * (src/gaussian_splats/training/train.py:137-138, the torch expression
 * (image.clamp(0, 1) - target).abs().mean() with clamp != 0, without the
 * clamp otherwise).  Writes loss[0] (fp32, deterministic) and code[numel]
 * int8 = sign(image' - target), 0 where the clamp stops the gradient, for
 * gs_l1_loss_bwd.  The workspace holds the per-workgroup partial sums. */
GS_API size_t gs_l1_loss_workspace_bytes(int64_t numel);
GS_API int gs_l1_loss_fwd(
    const float* image, const float* target, int64_t numel, int32_t clamp,
    float* loss, int8_t* code, void* workspace, size_t workspace_bytes,
    void* stream);

/* grad_image = code * (grad_loss[0] * (1 / numel)): autograd's gradient of
 * the expression above (train.py:151), with grad_loss in device memory. */
GS_API int gs_l1_loss_bwd(
    const int8_t* code, const float* grad_loss, int64_t numel,
    float* grad_image, void* stream);

/* Structural similarity term of the training step (train.py:139 through
 * training/utils.py:65-67: torchmetrics structural_similarity_index_measure
 * with data_range = 1 and its defaults, over the three channels of an
 * [H, W, 3] image).  gs_ssim_fwd writes the mean SSIM to ssim[0] and keeps
 * in the workspace what gs_ssim_bwd needs; gs_ssim_bwd writes
 * grad_image = grad_ssim[0] * d SSIM / d image (grad_ssim in device memory)
 * from the same image, target and workspace.  H and W must exceed 10. */
GS_API size_t gs_ssim_workspace_bytes(int32_t height, int32_t width);
GS_API int gs_ssim_fwd(
    const float* image, const float* target, int32_t height, int32_t width,
    float* ssim, void* workspace, size_t workspace_bytes, void* stream);
GS_API int gs_ssim_bwd(
    const float* image, const float* target, int32_t height, int32_t width,
    const float* grad_ssim, const void* workspace, size_t workspace_bytes,
    float* grad_image, void* stream);

/* Regularisers of the training step (train.py:140-141 before their
 * weights): out[0] = mean(sigmoid(opacity[N])), out[1] = mean(exp(scale[N,3])),
 * deterministic; the backward writes autograd's gradients of the two means
 * for the upstream gradients grad_out[2] (device memory). */
GS_API size_t gs_splat_regularizers_workspace_bytes(int64_t n);
GS_API int gs_splat_regularizers_fwd(
    const float* opacity, const float* scale, int64_t n, float* out,
    void* workspace, size_t workspace_bytes, void* stream);
GS_API int gs_splat_regularizers_bwd(
    const float* opacity, const float* scale, int64_t n, const float* grad_out,
    float* grad_opacity, float* grad_scale, void* stream);

/* One Adam step (torch.optim.Adam's update, multi-tensor path, no amsgrad)
 * over up to GS_ADAM_MAX_TENSORS float32 tensors in one launch: the optimiser
 * step of the training loop (src/gaussian_splats/training/train.py:115,151).
 * `step` is the step count after this step (1 on the first); `lr` is per
 * tensor (the reference changes the position group's rate every step,
 * train.py:131-133).  Updates param, exp_avg and exp_avg_sq in place. */
#define GS_ADAM_MAX_TENSORS 8
typedef struct gs_adam_tensor {
  float* param;
  const float* grad;
  float* exp_avg;
  float* exp_avg_sq;
  int64_t numel;
  double lr;
  int64_t step;
} gs_adam_tensor;
GS_API int gs_adam_step(
    const gs_adam_tensor* tensors, int32_t count, double beta1, double beta2,
    double eps, double weight_decay, void* stream);

/* Scene files: the binary PLY "vertex" records of a Gaussian-splat scene
 * (src/gaussian_splats/splats/ply.py).  Fields per Gaussian in canonical
 * order: mean 3, normals 3, rotation 4, scale 3, opacity 1, color 3K
 * (coefficient-major, RGB innermost) — 14 + 3K float32 values. */
#define GS_PLY_MAX_FIELDS 89 /* 14 + 3 * 25 (SH degree 4) */

/* Splits n records of record_bytes bytes each (device memory, 16-byte
 * aligned, the file's vertex block as stored) into the six parameter
 * tensors: output float j of a Gaussian (canonical order) is the float32 at
 * byte field_offsets[j] of its record (field_offsets in host memory, 14 +
 * 3 sh_coeffs entries), or 0 where the offset is -1; big_endian != 0 swaps
 * each value's bytes.  Replaces the per-property reads of load_ply
 * (ply.py:55-89), which the host's header parse turns into offsets. */
GS_API int gs_ply_unpack(
    const void* records, int64_t n, int32_t record_bytes,
    const int32_t* field_offsets, int32_t big_endian, int32_t sh_coeffs,
    float* mean, float* normals, float* rotation, float* scale, float* opacity,
    float* color, void* stream);

/* Writes n records of 14 + 3 sh_coeffs little-endian float32 values in the
 * property order of save_ply (ply.py:23-43): x y z nx ny nz f_dc_0..2
 * f_rest_0.. (f_rest_{c (K-1) + k - 1} = color[k][c]) opacity scale_0..2
 * rot_0..3.  normals may be NULL (zeros, as ply.py:20 substitutes). */
GS_API int gs_ply_pack(
    const float* mean, const float* normals, const float* rotation,
    const float* scale, const float* opacity, const float* color, int64_t n,
    int32_t sh_coeffs, void* records, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GS_RASTER_H */
