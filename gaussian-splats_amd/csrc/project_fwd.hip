// Projection stage: EWA 2-D covariance, SH colour, sigmoid opacity, tile
// rectangle and culled intersection count, one thread per Gaussian.
//
// Semantics follow src/gaussian_splats/splats/camera.py:81-124 (projection and
// Jacobian), splats/utils.py:8-75 (quaternion, SH), kernels/rasterize/torch.py:
// 165-203 (project), torch.py:206-252 (cull, extent, rectangle) and the
// original-index outputs of kernels/rasterize/project.py:234-253.
//
// This file is compiled with -ffp-contract=off: the tile rectangle is
// floor((u -/+ r) / tile) and must round exactly as the CPU restatement does.
#include <algorithm>
#include <cmath>

#include "common.h"
#include "sh.h"

namespace gs {
namespace {

constexpr int kProjectBlock = 256;

// One camera: world -> camera extrinsics and intrinsics, by value (kernel
// arguments).
struct FwdCamera {
  float r[9];
  float t[3];
  float fx, fy, cx, cy;
  float lim_x, lim_y;  // 1.3 * tan(half field of view), camera.py:106-116
  int tile_x, tile_y;  // the view's tile origin in a mosaic (0, 0 for one view)
};

constexpr int kMaxViews = 16;  // cameras per launch

struct ProjectArgs {
  const float* mean;
  const float* rotation;
  const float* scale;
  const float* opacity;
  const float* color;
  FwdCamera cam[kMaxViews];
  int views;  // view v's outputs start at Gaussian v * n
  int64_t n;
  float tile;
  float tiles_w, tiles_h;  // of one view
  float near_plane, far_plane, eps;
  int ellipsoid;
  float ellipsoid_extent;  // sqrt(-2 log1p(-confidence))
  float ellipsoid_cutoff;  // -2 log1p(-confidence)
  float* pmean;
  float* pinv;
  float* pcolor;
  float* popacity;
  int* bounds;           // optional with tile_rects
  int* counts;
  GsRecord* records;     // optional
  uint32_t* depth_keys;  // optional
  uint32_t* tile_rects;  // optional: packed rectangles (pack_rect) in mosaic tiles
};

// The colour block of kProjectBlock Gaussians is staged through LDS with
// coalesced 16-byte loads (sh::stage_block), then each thread reads its own
// K*3 coefficients from its row (sh::row_load; rows of sh::row_stride floats).
template <int K>
__global__ __launch_bounds__(kProjectBlock) void project_fwd_kernel(ProjectArgs a) {
  constexpr int F = 3 * K;
  constexpr int S = sh::row_stride<F>();
  __shared__ __align__(16) float coeff[kProjectBlock * S];

  const int64_t base = int64_t(blockIdx.x) * kProjectBlock;
  const int64_t nvalid = min(int64_t(kProjectBlock), a.n - base);
  const int64_t gi = base + threadIdx.x;
  const bool have = gi < a.n;
  // The thread's own parameters are requested before the colour block, so
  // their loads are in flight together with it (threads past the end read
  // the last Gaussian, branch-free, and return after the barrier).
  const int64_t gl = have ? gi : a.n - 1;
  const float mx = load_nt(a.mean + gl * 3 + 0);
  const float my = load_nt(a.mean + gl * 3 + 1);
  const float mz = load_nt(a.mean + gl * 3 + 2);
  const float4 q = load_nt(reinterpret_cast<const float4*>(a.rotation) + gl);
  const float ls0 = load_nt(a.scale + gl * 3 + 0);
  const float ls1 = load_nt(a.scale + gl * 3 + 1);
  const float ls2 = load_nt(a.scale + gl * 3 + 2);
  const float lo = load_nt(a.opacity + gl);
  sh::stage_block<F, kProjectBlock>(a.color + base * F, int(nvalid), coeff);
  __syncthreads();
  if (!have) return;

  // View-independent terms, computed once per Gaussian, in double precision
  // like the covariance chain they feed (see below).
  // Normalised quaternion (w, x, y, z) -> rotation (utils.py:8-25).
  const double dqx = q.x, dqy = q.y, dqz = q.z, dqw = q.w;
  const double qn = fmax(sqrt(dqx * dqx + dqy * dqy + dqz * dqz + dqw * dqw), 1e-12);
  const double qw = dqx / qn, qx = dqy / qn, qy = dqz / qn, qz = dqw / qn;
  const double q00 = 1.0 - 2.0 * (qy * qy + qz * qz);
  const double q01 = 2.0 * (qx * qy - qw * qz);
  const double q02 = 2.0 * (qx * qz + qw * qy);
  const double q10 = 2.0 * (qx * qy + qw * qz);
  const double q11 = 1.0 - 2.0 * (qx * qx + qz * qz);
  const double q12 = 2.0 * (qy * qz - qw * qx);
  const double q20 = 2.0 * (qx * qz - qw * qy);
  const double q21 = 2.0 * (qy * qz + qw * qx);
  const double q22 = 1.0 - 2.0 * (qx * qx + qy * qy);

  const double sx = exp(double(ls0));
  const double sy = exp(double(ls1));
  const double sz = exp(double(ls2));

  const float alpha0 = 1.0f / (1.0f + expf(-lo));
  // Extent of the ellipse in standard deviations (torch.py:233-252) and the
  // largest quadratic form D for which the blended alpha can reach 1/255.
  const float extent = a.ellipsoid ? a.ellipsoid_extent : 2.0f * sqrtf(logf(alpha0 * 255.0f));
  float cut;
  if (a.ellipsoid) {
    cut = alpha0 >= (1.0f / 255.0f) ? a.ellipsoid_cutoff : -1.0f;
  } else {
    cut = 2.0f * logf(alpha0 * 255.0f);
  }

  for (int view = 0; view < a.views; ++view) {
    const FwdCamera& cam = a.cam[view];
    const int64_t vi = int64_t(view) * a.n + gi;  // output slot
    const float r00 = cam.r[0], r01 = cam.r[1], r02 = cam.r[2];
    const float r10 = cam.r[3], r11 = cam.r[4], r12 = cam.r[5];
    const float r20 = cam.r[6], r21 = cam.r[7], r22 = cam.r[8];
    const float t0 = cam.t[0], t1 = cam.t[1], t2 = cam.t[2];

    // Camera-space point p = R mu + t (camera.py:94).
    const float px = r00 * mx + r01 * my + r02 * mz + t0;
    const float py = r10 * mx + r11 * my + r12 * mz + t1;
    const float pz = r20 * mx + r21 * my + r22 * mz + t2;
    // Depth along the viewing axis (-Z forward), kept at least 1e-4 from zero
    // (camera.py:96-97).
    const float d = -pz;
    const float dc = fabsf(d) >= 1e-4f ? d : copysignf(1e-4f, d);

    // Pixel coordinates use the unclamped depth, as the homogeneous divide of
    // camera.py:101-102 does; the Jacobian below uses the clamped one.
    const float u = cam.fx * px / d + cam.cx;
    const float v = -cam.fy * py / d + cam.cy;

    // The 2-D covariance and its inverse, in double precision from the
    // float32 inputs.  For a nearly degenerate covariance (an edge-on flat
    // splat, a needle) det = c00 c11 - c01^2 cancels, and float32 arithmetic
    // loses the condition number's worth of digits in the inverse; computed
    // in double, the stored inverse is the float32 rounding of the exact
    // value.  The projection backward recomputes the same chain in double.
    // Perspective Jacobian with the 1.3 x half-FOV clamp (camera.py:106-119),
    // at the camera-space point p = R mu + t recomputed in double.
    const double dpx = double(r00) * mx + double(r01) * my + double(r02) * mz + double(t0);
    const double dpy = double(r10) * mx + double(r11) * my + double(r12) * mz + double(t1);
    const double dpz = double(r20) * mx + double(r21) * my + double(r22) * mz + double(t2);
    const double dd = -dpz;
    const double ddc = fabs(dd) >= 1e-4 ? dd : copysign(1e-4, dd);
    const double nx = fmin(fmax(dpx / ddc, -double(cam.lim_x)), double(cam.lim_x));
    const double ny = fmin(fmax(dpy / ddc, -double(cam.lim_y)), double(cam.lim_y));
    const double j00 = double(cam.fx) / ddc;
    const double j02 = double(cam.fx) * nx / ddc;
    const double j11 = -double(cam.fy) / ddc;
    const double j12 = -double(cam.fy) * ny / ddc;
    // W = J Rc.
    const double w00 = j00 * r00 + j02 * r20;
    const double w01 = j00 * r01 + j02 * r21;
    const double w02 = j00 * r02 + j02 * r22;
    const double w10 = j11 * r10 + j12 * r20;
    const double w11 = j11 * r11 + j12 * r21;
    const double w12 = j11 * r12 + j12 * r22;

    // M = W Rq diag(s); Sigma = M M^T + eps I (camera.py:121-123).
    const double m00 = (w00 * q00 + w01 * q10 + w02 * q20) * sx;
    const double m01 = (w00 * q01 + w01 * q11 + w02 * q21) * sy;
    const double m02 = (w00 * q02 + w01 * q12 + w02 * q22) * sz;
    const double m10 = (w10 * q00 + w11 * q10 + w12 * q20) * sx;
    const double m11 = (w10 * q01 + w11 * q11 + w12 * q21) * sy;
    const double m12 = (w10 * q02 + w11 * q12 + w12 * q22) * sz;
    const double c00 = m00 * m00 + m01 * m01 + m02 * m02 + double(a.eps);
    const double c01 = m00 * m10 + m01 * m11 + m02 * m12;
    const double c11 = m10 * m10 + m11 * m11 + m12 * m12 + double(a.eps);
    const double rdet = 1.0 / (c00 * c11 - c01 * c01);
    const float i00 = float(c11 * rdet);
    const float i01 = float(-c01 * rdet);
    const float i11 = float(c00 * rdet);

    // View direction from the Gaussian to the camera centre -R^T t
    // (torch.py:198, camera.py:37-39).
    const float ex = -(r00 * t0 + r10 * t1 + r20 * t2) - mx;
    const float ey = -(r01 * t0 + r11 * t1 + r21 * t2) - my;
    const float ez = -(r02 * t0 + r12 * t1 + r22 * t2) - mz;
    const float en = fmaxf(sqrtf(ex * ex + ey * ey + ez * ez), 1e-12f);
    float basis[K];
    sh::basis<K>(ex / en, ey / en, ez / en, basis);
    float coef[F];
    sh::row_load<F>(coeff, threadIdx.x, coef);
    float rgb[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < K; ++k) acc += basis[k] * coef[k * 3 + c];
      rgb[c] = fmaxf(acc + 0.5f, 0.0f);  // utils.py:75
    }

    // Rectangle of tiles touched by the extent ellipse (torch.py:233-252).
    const float rx = extent * sqrtf(float(c00));
    const float ry = extent * sqrtf(float(c11));
    // fmaxf/fminf map a NaN extent (alpha0 < 1/255) to the empty rectangle [0, 0).
    const float bx0 = fminf(fmaxf(floorf((u - rx) / a.tile), 0.0f), a.tiles_w);
    const float bx1 = fminf(fmaxf(floorf((u + rx) / a.tile) + 1.0f, 0.0f), a.tiles_w);
    const float by0 = fminf(fmaxf(floorf((v - ry) / a.tile), 0.0f), a.tiles_h);
    const float by1 = fminf(fmaxf(floorf((v + ry) / a.tile) + 1.0f, 0.0f), a.tiles_h);
    const int x0 = int(bx0), x1 = int(bx1), y0 = int(by0), y1 = int(by1);
    const bool visible = dc > a.near_plane && dc < a.far_plane;
    const int count = visible ? (x1 - x0) * (y1 - y0) : 0;

    a.pmean[vi * 3 + 0] = u;
    a.pmean[vi * 3 + 1] = v;
    a.pmean[vi * 3 + 2] = dc;
    reinterpret_cast<float4*>(a.pinv)[vi] = make_float4(i00, i01, i01, i11);
    a.pcolor[vi * 3 + 0] = rgb[0];
    a.pcolor[vi * 3 + 1] = rgb[1];
    a.pcolor[vi * 3 + 2] = rgb[2];
    a.popacity[vi] = alpha0;
    if (a.bounds)
      reinterpret_cast<int4*>(a.bounds)[vi] =
          make_int4(x0 + cam.tile_x, x1 + cam.tile_x, y0 + cam.tile_y, y1 + cam.tile_y);
    a.counts[vi] = count;
    if (a.tile_rects)
      a.tile_rects[vi] =
          count > 0 ? pack_rect(x0 + cam.tile_x, x1 - x0, y0 + cam.tile_y, y1 - y0) : kNoRect;

    if (a.records) {
      float4* rec = reinterpret_cast<float4*>(a.records + vi);
      rec[0] = make_float4(u, v, alpha0, dc);
      rec[1] = make_float4(i00, i01, i11, cut);
      rec[2] = make_float4(rgb[0], rgb[1], rgb[2], 0.0f);
    }
    if (a.depth_keys) a.depth_keys[vi] = count > 0 ? __float_as_uint(dc) : 0xFFFFFFFFu;
  }
}

__global__ __launch_bounds__(256) void pack_records_kernel(
    const float* __restrict__ pmean, const float* __restrict__ pinv,
    const float* __restrict__ pcolor, const float* __restrict__ popacity, int64_t n,
    int ellipsoid, float ellipsoid_cutoff, GsRecord* __restrict__ records) {
  const int64_t gi = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gi >= n) return;
  const float alpha0 = popacity[gi];
  float cut;
  if (ellipsoid) {
    cut = alpha0 >= (1.0f / 255.0f) ? ellipsoid_cutoff : -1.0f;
  } else {
    cut = 2.0f * logf(alpha0 * 255.0f);
  }
  const float4 inv = reinterpret_cast<const float4*>(pinv)[gi];
  float4* rec = reinterpret_cast<float4*>(records + gi);
  rec[0] = make_float4(pmean[gi * 3], pmean[gi * 3 + 1], alpha0, pmean[gi * 3 + 2]);
  rec[1] = make_float4(inv.x, inv.y, inv.w, cut);
  rec[2] = make_float4(pcolor[gi * 3], pcolor[gi * 3 + 1], pcolor[gi * 3 + 2], 0.0f);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace gs

using namespace gs;

namespace {

// Projects for `views` cameras (host arrays: rotations [V, 9], translations
// [V, 3], optional intrinsics [V, 4] = fx, fy, cx, cy, else the view's) in
// launches of up to kMaxViews cameras.  With `mosaic`, bounds and tile
// rectangles are shifted to each view's tile origin in the mosaic of `view`.
int project_views(const float* mean, const float* rotation, const float* scale,
                  const float* opacity, const float* color, int64_t n, int32_t num_sh,
                  const float* camera_rotations, const float* camera_translations,
                  const float* intrinsics, int views, gs_view view, bool mosaic,
                  float* projected_mean, float* inverse_covariance, float* projected_color,
                  float* projected_opacity, int32_t* bounds, int32_t* counts, void* records,
                  uint32_t* depth_keys, uint32_t* tile_rects, void* stream) {
  GS_REQUIRE(n >= 0, GS_ERR_INVALID_ARGUMENT, "negative Gaussian count");
  GS_TRY(check_view(view, true));
  GS_REQUIRE(num_sh == 1 || num_sh == 4 || num_sh == 9 || num_sh == 16, GS_ERR_UNSUPPORTED,
             "SH degrees above 3 are not implemented (got %d coefficients)", num_sh);
  if (n == 0) return GS_OK;
  GS_REQUIRE(mean && rotation && scale && opacity && color && camera_rotations &&
                 camera_translations && projected_mean && inverse_covariance &&
                 projected_color && projected_opacity && (bounds || tile_rects) && counts,
             GS_ERR_INVALID_ARGUMENT, "null pointer argument");
  GS_REQUIRE(aligned16(rotation) && aligned16(color) && aligned16(inverse_covariance) &&
                 (!bounds || aligned16(bounds)) && (!records || aligned16(records)),
             GS_ERR_INVALID_ARGUMENT,
             "rotation, color, inverse_covariance, bounds and records must be 16-byte aligned");
  GS_REQUIRE(int64_t(views) * n < (int64_t(1) << 31), GS_ERR_OVERFLOW,
             "too many Gaussians (%lld x %d views)", (long long)n, views);

  ProjectArgs a;
  a.mean = mean;
  a.rotation = rotation;
  a.scale = scale;
  a.opacity = opacity;
  a.color = color;
  a.n = n;
  a.tile = float(view.tile_size);
  a.tiles_w = float(tiles_along(view.image_width, view.tile_size));
  a.tiles_h = float(tiles_along(view.image_height, view.tile_size));
  a.near_plane = view.near_plane;
  a.far_plane = view.far_plane;
  a.eps = view.covariance_epsilon;
  a.ellipsoid = view.rendering_mode == GS_MODE_ELLIPSOID;
  const double cutoff = -2.0 * std::log1p(-double(view.confidence));
  a.ellipsoid_cutoff = float(cutoff);
  a.ellipsoid_extent = float(std::sqrt(cutoff));
  const Mosaic m = mosaic_of(view);
  GS_REQUIRE(!tile_rects || ((mosaic ? m.tiles_w() : m.tw) <= kMaxAxisTiles &&
                             (mosaic ? m.tiles_h() : m.th) <= kMaxAxisTiles),
             GS_ERR_UNSUPPORTED, "packed tile rectangles need at most %d x %d tiles",
             kMaxAxisTiles, kMaxAxisTiles);
  const dim3 grid(unsigned(ceil_div(n, kProjectBlock)));
  hipStream_t s = as_stream(stream);
  for (int first = 0; first < views; first += kMaxViews) {
    a.views = std::min(kMaxViews, views - first);
    for (int j = 0; j < a.views; ++j) {
      const int vw = first + j;
      FwdCamera& c = a.cam[j];
      // Host memory: the cameras travel as kernel arguments.
      for (int i = 0; i < 9; ++i) c.r[i] = camera_rotations[vw * 9 + i];
      for (int i = 0; i < 3; ++i) c.t[i] = camera_translations[vw * 3 + i];
      const float* k = intrinsics ? intrinsics + vw * 4 : nullptr;
      c.fx = k ? k[0] : view.fx;
      c.fy = k ? k[1] : view.fy;
      c.cx = k ? k[2] : view.cx;
      c.cy = k ? k[3] : view.cy;
      // Same double-precision expression as camera.py:106-116, rounded once to fp32.
      c.lim_x = float(1.3 * (double(view.image_width) / (2.0 * double(c.fx))));
      c.lim_y = float(1.3 * (double(view.image_height) / (2.0 * double(c.fy))));
      c.tile_x = mosaic ? (vw % m.cols) * m.tw : 0;
      c.tile_y = mosaic ? (vw / m.cols) * m.th : 0;
    }
    const int64_t off = int64_t(first) * n;  // first output slot of this launch
    a.pmean = projected_mean + off * 3;
    a.pinv = inverse_covariance + off * 4;
    a.pcolor = projected_color + off * 3;
    a.popacity = projected_opacity + off;
    a.bounds = bounds ? bounds + off * 4 : nullptr;
    a.counts = counts + off;
    a.tile_rects = tile_rects ? tile_rects + off : nullptr;
    a.records = records ? static_cast<GsRecord*>(records) + off : nullptr;
    a.depth_keys = depth_keys ? depth_keys + off : nullptr;
    switch (num_sh) {
      case 1: launch_timed(project_fwd_kernel<1>, grid, kProjectBlock, 0, s, a); break;
      case 4: launch_timed(project_fwd_kernel<4>, grid, kProjectBlock, 0, s, a); break;
      case 9: launch_timed(project_fwd_kernel<9>, grid, kProjectBlock, 0, s, a); break;
      default: launch_timed(project_fwd_kernel<16>, grid, kProjectBlock, 0, s, a); break;
    }
    GS_TRY(check_launch("project_fwd"));
  }
  return GS_OK;
}

}  // namespace

extern "C" GS_API int gs_project_and_count(
    const float* mean, const float* rotation, const float* scale, const float* opacity,
    const float* color, int64_t n, int32_t num_sh, const float* camera_rotation,
    const float* camera_translation, gs_view view, float* projected_mean,
    float* inverse_covariance, float* projected_color, float* projected_opacity,
    int32_t* bounds, int32_t* counts, void* records, uint32_t* depth_keys, uint32_t* tile_rects,
    void* stream) {
  clear_error();
  return project_views(mean, rotation, scale, opacity, color, n, num_sh, camera_rotation,
                       camera_translation, nullptr, 1, view, false, projected_mean,
                       inverse_covariance, projected_color, projected_opacity, bounds, counts,
                       records, depth_keys, tile_rects, stream);
}

extern "C" GS_API int gs_project_views(
    const float* mean, const float* rotation, const float* scale, const float* opacity,
    const float* color, int64_t n, int32_t num_sh, const float* camera_rotations,
    const float* camera_translations, const float* intrinsics, gs_view view,
    float* projected_mean, float* inverse_covariance, float* projected_color,
    float* projected_opacity, int32_t* bounds, int32_t* counts, void* records,
    uint32_t* depth_keys, uint32_t* tile_rects, void* stream) {
  clear_error();
  return project_views(mean, rotation, scale, opacity, color, n, num_sh, camera_rotations,
                       camera_translations, intrinsics, mosaic_of(view).views, view, true,
                       projected_mean, inverse_covariance, projected_color, projected_opacity,
                       bounds, counts, records, depth_keys, tile_rects, stream);
}

extern "C" GS_API int gs_pack_records(const float* projected_mean,
                                      const float* inverse_covariance,
                                      const float* projected_color,
                                      const float* projected_opacity, int64_t n, gs_view view,
                                      void* records, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0, GS_ERR_INVALID_ARGUMENT, "negative Gaussian count");
  if (n == 0) return GS_OK;
  GS_REQUIRE(projected_mean && inverse_covariance && projected_color && projected_opacity &&
                 records,
             GS_ERR_INVALID_ARGUMENT, "null pointer argument");
  GS_REQUIRE(aligned16(inverse_covariance) && aligned16(records), GS_ERR_INVALID_ARGUMENT,
             "inverse_covariance and records must be 16-byte aligned");
  const double cutoff = -2.0 * std::log1p(-double(view.confidence));
  pack_records_kernel<<<unsigned(ceil_div(n, 256)), 256, 0, as_stream(stream)>>>(
      projected_mean, inverse_covariance, projected_color, projected_opacity, n,
      view.rendering_mode == GS_MODE_ELLIPSOID, float(cutoff), static_cast<GsRecord*>(records));
  return check_launch("pack_records");
}
