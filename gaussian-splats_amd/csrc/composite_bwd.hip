// Backward compositing: one wave64 per tile, back-to-front over the entries
// each pixel processed while active (positions < n_contributors).
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
// Per Gaussian, each lane sums over its pixels the factors that do not
// depend on the Gaussian (q = dL/dalpha * G, q dx, q dy, q dx^2, q dx dy,
// q dy^2 and g T alpha); the wave reduces them with DPP row operations, and
// one 9-lane fp32 atomic add writes
//   (u, v, inv00, inv01, inv11, r, g, b, opacity) += (-2 k (a Sx + b Sy),
//   -2 k (b Sx + c Sy), k Sxx, k Sxy, k Syy, Sr, Sg, Sb, Sq),  k = -o / 2,
// once per (tile, Gaussian).  Replaces composite_bwd.py:47-204 and the
// index_add_ scatter of composite_bwd.py:268-273.
#include "common.h"
#include "raster_math.h"

namespace gs {
namespace {

constexpr int kWavesPerBlock = 4;

struct CompositeBwdArgs {
  const float* pmean;
  const float* pinv;
  const float* pcolor;
  const float* popacity;
  const int32_t* ids;
  const int64_t* ranges;
  const float* grad_image;
  const float* final_t;
  const int32_t* n_contrib;
  int width, height, tiles_w, num_tiles;
  float* grad;  // [N, 9]
};

template <int TILE>
__global__ __launch_bounds__(kWavesPerBlock * 64) void composite_bwd_kernel(CompositeBwdArgs a) {
  constexpr int NPIX = TILE * TILE;
  constexpr int PIX = NPIX >= 64 ? NPIX / 64 : 1;
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int tile = xcd_swizzle(blockIdx.x, gridDim.x) * kWavesPerBlock + wid;
  if (tile >= a.num_tiles) return;

  const int tx = tile % a.tiles_w;
  const int ty = tile / a.tiles_w;
  const int ox = tx * TILE, oy = ty * TILE;
  const int64_t start = a.ranges[2 * tile];

  float pxf[PIX], pyf[PIX];
  float T[PIX], gr[PIX], gg[PIX], gb[PIX], gs_[PIX];
  int ncon[PIX];
  int max_n = 0;
#pragma unroll
  for (int k = 0; k < PIX; ++k) {
    const int q = lane + 64 * k;
    const int px = ox + (q % TILE), py = oy + (q / TILE);
    const bool valid = q < NPIX && px < a.width && py < a.height;
    const int64_t pix = int64_t(py) * a.width + px;
    pxf[k] = float(px);
    pyf[k] = float(py);
    T[k] = valid ? a.final_t[pix] : 1.0f;
    ncon[k] = valid ? a.n_contrib[pix] : 0;
    gr[k] = valid ? a.grad_image[pix * 3 + 0] : 0.0f;
    gg[k] = valid ? a.grad_image[pix * 3 + 1] : 0.0f;
    gb[k] = valid ? a.grad_image[pix * 3 + 2] : 0.0f;
    gs_[k] = 0.0f;
    max_n = max(max_n, ncon[k]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) max_n = max(max_n, __shfl_xor(max_n, o, 64));

  const float rx0 = float(ox), ry0 = float(oy);
  const float rx1 = float(min(ox + TILE, a.width) - 1);
  const float ry1 = float(min(oy + TILE, a.height) - 1);

  for (int64_t top = start + max_n; top > start; top -= 64) {
    const int64_t e = top - 1 - lane;
    LaneSplat mine;
    int gid = 0;
    bool keep = false;
    if (e >= start) {
      gid = a.ids[e];
      const GsRecord rec = load_projected(a.pmean, a.pinv, a.pcolor, a.popacity, gid);
      keep = touches_rect(rec, rx0, rx1, ry0, ry1);
      mine = lane_splat(rec);
    }
    uint64_t mask = __ballot(keep);
    while (mask) {
      const int j = __builtin_ctzll(mask);
      mask &= mask - 1;
      const Splat s = broadcast(mine, j);
      const int pos = int(top - 1 - start) - j;
      float sq = 0.0f, sx = 0.0f, sy = 0.0f, sxx = 0.0f, sxy = 0.0f, syy = 0.0f;
      float sr = 0.0f, sg = 0.0f, sb = 0.0f;
      bool touched = false;
      // Branch-free: an entry a pixel did not process while active, or whose
      // alpha is cut to 0, runs with alpha = 0, which leaves T, g.S and every
      // sum unchanged.
#pragma unroll
      for (int k = 0; k < PIX; ++k) {
        const float dx = pxf[k] - s.u;
        const float dy = pyf[k] - s.v;
        float prob;
        const float raw = raw_alpha<false>(s, dx, dy, prob);
        const float alpha = pos < ncon[k] ? blend_alpha(raw) : 0.0f;
        const bool hit = alpha > 0.0f;
        touched |= hit;
        const float t_before = hit ? T[k] * __builtin_amdgcn_rcpf(1.0f - alpha) : T[k];
        const float w = t_before * alpha;
        sr += gr[k] * w;
        sg += gg[k] * w;
        sb += gb[k] * w;
        const float gc = gr[k] * s.r + gg[k] * s.g + gb[k] * s.bl;
        const float diff = gc - gs_[k];
        gs_[k] += alpha * diff;
        T[k] = t_before;
        const float q = (hit && raw <= kMaxAlpha) ? t_before * diff * prob : 0.0f;
        const float qx = q * dx;
        const float qy = q * dy;
        sq += q;
        sx += qx;
        sy += qy;
        sxx += qx * dx;
        sxy += qx * dy;
        syy += qy * dy;
      }
      if (__ballot(touched) == 0) continue;
      sq = wave_sum_lane63(sq);
      sx = wave_sum_lane63(sx);
      sy = wave_sum_lane63(sy);
      sxx = wave_sum_lane63(sxx);
      sxy = wave_sum_lane63(sxy);
      syy = wave_sum_lane63(syy);
      sr = wave_sum_lane63(sr);
      sg = wave_sum_lane63(sg);
      sb = wave_sum_lane63(sb);
      // Gaussian constants, uniform across the wave.
      const float k = -0.5f * s.o;
      const float ga = bcast(mine.a, j), gbb = bcast(mine.bb, j), gcc = bcast(mine.c, j);
      const float tq = bcast(sq, 63), tx_ = bcast(sx, 63), ty_ = bcast(sy, 63);
      const float txx = bcast(sxx, 63), txy = bcast(sxy, 63), tyy = bcast(syy, 63);
      const float tr = bcast(sr, 63), tg = bcast(sg, 63), tb = bcast(sb, 63);
      // Lane i of `val` carries field i of the 9-float gradient row.
      float val = tq;
      val = write_lane(val, -2.0f * k * (ga * tx_ + gbb * ty_), 0);
      val = write_lane(val, -2.0f * k * (gbb * tx_ + gcc * ty_), 1);
      val = write_lane(val, k * txx, 2);
      val = write_lane(val, k * txy, 3);
      val = write_lane(val, k * tyy, 4);
      val = write_lane(val, tr, 5);
      val = write_lane(val, tg, 6);
      val = write_lane(val, tb, 7);
      if (lane < 9) {
        const int g = __builtin_amdgcn_readlane(gid, j);
        unsafeAtomicAdd(a.grad + int64_t(g) * 9 + lane, val);
      }
    }
  }
}

template <int TILE>
void launch(const CompositeBwdArgs& a, hipStream_t s) {
  const unsigned blocks = unsigned(ceil_div(a.num_tiles, kWavesPerBlock));
  composite_bwd_kernel<TILE><<<blocks, kWavesPerBlock * 64, 0, s>>>(a);
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" GS_API int gs_composite_bwd(const float* projected_mean,
                                       const float* inverse_covariance,
                                       const float* projected_color,
                                       const float* projected_opacity,
                                       const int32_t* gaussian_ids, const int64_t* ranges,
                                       const float* grad_image, const float* final_transmittance,
                                       const int32_t* n_contributors, gs_view view,
                                       float* grad_projected, void* stream) {
  clear_error();
  GS_TRY(check_view(view, true));
  GS_REQUIRE(view.rendering_mode == GS_MODE_GAUSSIAN, GS_ERR_UNSUPPORTED,
             "Backward gradients are only supported for Gaussian rendering.");
  GS_REQUIRE(ranges && grad_image && final_transmittance && n_contributors && grad_projected,
             GS_ERR_INVALID_ARGUMENT, "null pointer argument");
  GS_REQUIRE((reinterpret_cast<uintptr_t>(inverse_covariance) & 15u) == 0,
             GS_ERR_INVALID_ARGUMENT, "inverse_covariance must be 16-byte aligned");
  CompositeBwdArgs a;
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
  a.tiles_w = tiles_along(view.image_width, view.tile_size);
  a.num_tiles = a.tiles_w * tiles_along(view.image_height, view.tile_size);
  a.grad = grad_projected;
  hipStream_t s = as_stream(stream);
  switch (view.tile_size) {
    case 4: launch<4>(a, s); break;
    case 8: launch<8>(a, s); break;
    case 16: launch<16>(a, s); break;
    default: launch<32>(a, s); break;
  }
  return check_launch("composite_bwd");
}
