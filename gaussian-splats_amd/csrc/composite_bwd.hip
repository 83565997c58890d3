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
// inputs <= 0.99).  Per Gaussian the nine partials (u, v, inv00, inv01, inv11,
// r, g, b, opacity) are summed over the lane's pixels, reduced across the wave
// and added once per (tile, Gaussian) with hardware fp32 atomics.
// Replaces composite_bwd.py:47-277 (which stores per-intersection rows and
// scatter-adds them with index_add_).
#include "block_scan.h"
#include "common.h"
#include "raster_math.h"

namespace gs {
namespace {

constexpr int kWavesPerBlock = 4;

struct CompositeBwdArgs {
  const GsRecord* records;
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
  float T[PIX], gr[PIX], gg[PIX], gb[PIX], sr[PIX], sg[PIX], sb[PIX];
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
    sr[k] = sg[k] = sb[k] = 0.0f;
    max_n = max(max_n, ncon[k]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) max_n = max(max_n, __shfl_xor(max_n, o, 64));

  const float rx0 = float(ox), ry0 = float(oy);
  const float rx1 = float(min(ox + TILE, a.width) - 1);
  const float ry1 = float(min(oy + TILE, a.height) - 1);

  for (int64_t top = start + max_n; top > start; top -= 64) {
    const int64_t e = top - 1 - lane;
    GsRecord rec;
    int gid = 0;
    bool keep = false;
    if (e >= start) {
      gid = a.ids[e];
      rec = load_record(a.records, gid);
      keep = touches_rect(rec, rx0, rx1, ry0, ry1);
    }
    uint64_t mask = __ballot(keep);
    while (mask) {
      const int j = __builtin_ctzll(mask);
      mask &= mask - 1;
      const Splat s = broadcast(rec, j);
      const int pos = int(top - 1 - start) - j;
      float acc[9];
#pragma unroll
      for (int i = 0; i < 9; ++i) acc[i] = 0.0f;
      bool touched = false;
#pragma unroll
      for (int k = 0; k < PIX; ++k) {
        if (pos >= ncon[k]) continue;
        const float dx = pxf[k] - s.u;
        const float dy = pyf[k] - s.v;
        float prob;
        const float raw = raw_alpha<false>(s, quad_form(s, dx, dy), prob);
        const float alpha = blend_alpha(raw);
        if (alpha == 0.0f) continue;
        touched = true;
        const float one_minus = 1.0f - alpha;
        const float t_before = T[k] * __builtin_amdgcn_rcpf(one_minus);
        const float w = t_before * alpha;
        acc[5] += gr[k] * w;
        acc[6] += gg[k] * w;
        acc[7] += gb[k] * w;
        const float dalpha =
            t_before * (gr[k] * (s.r - sr[k]) + gg[k] * (s.g - sg[k]) + gb[k] * (s.bl - sb[k]));
        sr[k] = alpha * s.r + one_minus * sr[k];
        sg[k] = alpha * s.g + one_minus * sg[k];
        sb[k] = alpha * s.bl + one_minus * sb[k];
        T[k] = t_before;
        if (raw <= kMaxAlpha) {
          acc[8] += dalpha * prob;
          // dL/dD = dalpha * o * dG/dD = -0.5 * dalpha * o * G.
          const float dD = -0.5f * dalpha * s.o * prob;
          acc[0] += -2.0f * dD * (s.a * dx + s.b * dy);
          acc[1] += -2.0f * dD * (s.b * dx + s.c * dy);
          acc[2] += dD * dx * dx;
          acc[3] += dD * dx * dy;
          acc[4] += dD * dy * dy;
        }
      }
      if (__ballot(touched) == 0) continue;
#pragma unroll
      for (int i = 0; i < 9; ++i) acc[i] = wave_sum(acc[i]);
      if (lane == 0) {
        const int g = __builtin_amdgcn_readlane(gid, j);
        float* dst = a.grad + int64_t(g) * 9;
#pragma unroll
        for (int i = 0; i < 9; ++i) unsafeAtomicAdd(dst + i, acc[i]);
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

extern "C" GS_API int gs_composite_bwd(const void* records, const int32_t* gaussian_ids,
                                       const int64_t* ranges, const float* grad_image,
                                       const float* final_transmittance,
                                       const int32_t* n_contributors, gs_view view,
                                       float* grad_projected, void* stream) {
  clear_error();
  GS_TRY(check_view(view, true));
  GS_REQUIRE(view.rendering_mode == GS_MODE_GAUSSIAN, GS_ERR_UNSUPPORTED,
             "Backward gradients are only supported for Gaussian rendering.");
  GS_REQUIRE(ranges && grad_image && final_transmittance && n_contributors && grad_projected,
             GS_ERR_INVALID_ARGUMENT, "null pointer argument");
  GS_REQUIRE((reinterpret_cast<uintptr_t>(records) & 15u) == 0, GS_ERR_INVALID_ARGUMENT,
             "records must be 16-byte aligned");
  CompositeBwdArgs a;
  a.records = static_cast<const GsRecord*>(records);
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
