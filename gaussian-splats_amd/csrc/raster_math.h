// Per-pixel compositing math shared by the forward and backward kernels, so both
// evaluate bit-identical alphas.
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace gs {

constexpr float kMinAlpha = 1.0f / 255.0f;  // torch.py:350, composite.py:82
constexpr float kMaxAlpha = 0.99f;          // torch.py:349, composite.py:81
constexpr float kNegHalfLog2e = -0.72134752044448170f;  // -0.5 / ln 2

// Gaussian broadcast to every lane of a wave (values live in SGPRs).  The
// conic is pre-scaled so that exp(-D/2) = exp2(pa dx^2 + pb dx dy + pc dy^2)
// with D the quadratic form a dx^2 + 2 b dx dy + c dy^2 of utils.py:78-87.
struct Splat {
  float u, v, o, pa, pb, pc, cut, r, g, bl;
};

// Per-lane view of a gathered record with the pre-scaled conic.
struct LaneSplat {
  float u, v, o, pa, pb, pc, cut, r, g, b;
  float a, bb, c;  // unscaled inverse covariance (for the mean gradient)
};

__device__ __forceinline__ LaneSplat lane_splat(const GsRecord& r) {
  LaneSplat s;
  s.u = r.u;
  s.v = r.v;
  s.o = r.opacity;
  s.pa = kNegHalfLog2e * r.inv00;
  s.pb = (2.0f * kNegHalfLog2e) * r.inv01;
  s.pc = kNegHalfLog2e * r.inv11;
  s.cut = r.cut;
  s.r = r.r;
  s.g = r.g;
  s.b = r.b;
  s.a = r.inv00;
  s.bb = r.inv01;
  s.c = r.inv11;
  return s;
}

// log2 of the Gaussian falloff at pixel offset (dx, dy).
__device__ __forceinline__ float falloff_log2(const Splat& s, float dx, float dy) {
  return dx * (s.pa * dx + s.pb * dy) + s.pc * (dy * dy);
}

// Unclamped alpha = opacity * probability (utils.py:90-99); `prob` returns the
// probability.  Ellipsoid mode compares D = power / (-0.5 log2 e) with the
// cutoff stored in the record.
template <bool ELLIPSOID>
__device__ __forceinline__ float raw_alpha(const Splat& s, float dx, float dy, float& prob) {
  const float power = falloff_log2(s, dx, dy);
  if constexpr (ELLIPSOID) {
    prob = power >= kNegHalfLog2e * s.cut ? 1.0f : 0.0f;
  } else {
    prob = __builtin_amdgcn_exp2f(power);
  }
  return s.o * prob;
}

// Clamp to 0.99 and drop alphas below 1/255 (torch.py:349-350).
__device__ __forceinline__ float blend_alpha(float raw) {
  const float a = fminf(raw, kMaxAlpha);
  return a >= kMinAlpha ? a : 0.0f;
}

// Smallest value of the quadratic form over the pixel rectangle
// [x0, x1] x [y0, y1] (continuous, so no larger than over the integer pixels).
// The form is positive definite, so the minimum is 0 when the mean is inside
// and otherwise lies on an edge, where it is the clamped vertex of a parabola.
__device__ __forceinline__ float min_quad_over_rect(float a, float b, float c, float u, float v,
                                                    float x0, float x1, float y0, float y1) {
  const float lx = x0 - u, hx = x1 - u, ly = y0 - v, hy = y1 - v;
  if (lx <= 0.0f && hx >= 0.0f && ly <= 0.0f && hy >= 0.0f) return 0.0f;
  if (!(a > 0.0f) || !(c > 0.0f)) return 0.0f;  // degenerate: never skip
  float best = 3.0e38f;
  const float ex[2] = {lx, hx};
  const float ey[2] = {ly, hy};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float dx = ex[i];
    const float dy = fminf(fmaxf(-b * dx / c, ly), hy);
    best = fminf(best, a * dx * dx + 2.0f * b * dx * dy + c * dy * dy);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float dy = ey[i];
    const float dx = fminf(fmaxf(-b * dy / a, lx), hx);
    best = fminf(best, a * dx * dx + 2.0f * b * dx * dy + c * dy * dy);
  }
  return best;
}

// True when the Gaussian can reach alpha >= 1/255 somewhere in the rectangle.
// `cut` is the largest quadratic form with alpha >= 1/255 (2 ln(255 o) in
// Gaussian mode); the relative margin keeps the test conservative against the
// rounding of the per-pixel evaluation.  A skipped Gaussian has alpha == 0 at
// every pixel of the tile, so skipping changes neither colour nor
// transmittance; positions in the tile list are still counted.
__device__ __forceinline__ bool touches_rect(const GsRecord& r, float x0, float x1, float y0,
                                             float y1) {
  if (!(r.cut >= 0.0f)) return false;
  const float m = min_quad_over_rect(r.inv00, r.inv01, r.inv11, r.u, r.v, x0, x1, y0, y1);
  return m <= r.cut * (1.0f + 1e-3f) + 1e-3f;
}

__device__ __forceinline__ GsRecord load_record(const GsRecord* __restrict__ recs, int g) {
  const float4* p = reinterpret_cast<const float4*>(recs + g);
  const float4 a = p[0], b = p[1], c = p[2];
  GsRecord r;
  r.u = a.x;
  r.v = a.y;
  r.opacity = a.z;
  r.depth = a.w;
  r.inv00 = b.x;
  r.inv01 = b.y;
  r.inv11 = b.z;
  r.cut = b.w;
  r.r = c.x;
  r.g = c.y;
  r.b = c.z;
  r.pad = c.w;
  return r;
}

// Gathers the same fields from the op's projected outputs (projected_mean,
// inverse_covariance, projected_color, projected_opacity).  `cut` is computed
// with the expression project_fwd uses, so it is bit-identical to the record's.
__device__ __forceinline__ GsRecord load_projected(const float* __restrict__ pmean,
                                                   const float* __restrict__ pinv,
                                                   const float* __restrict__ pcolor,
                                                   const float* __restrict__ popacity, int g) {
  GsRecord r;
  const int64_t g3 = int64_t(g) * 3;
  r.u = pmean[g3];
  r.v = pmean[g3 + 1];
  r.depth = pmean[g3 + 2];
  const float4 inv = reinterpret_cast<const float4*>(pinv)[g];
  r.inv00 = inv.x;
  r.inv01 = inv.y;
  r.inv11 = inv.w;
  r.r = pcolor[g3];
  r.g = pcolor[g3 + 1];
  r.b = pcolor[g3 + 2];
  r.opacity = popacity[g];
  r.cut = 2.0f * logf(r.opacity * 255.0f);
  r.pad = 0.0f;
  return r;
}

__device__ __forceinline__ float bcast(float x, int j) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j));
}

// Returns `v` with lane `lane` replaced by the wave-uniform value `x`.
__device__ __forceinline__ float write_lane(float v, float x, int lane) {
  return __lane_id() == lane ? x : v;
}

// Broadcasts lane j's splat to the whole wave (v_readlane into SGPRs, so the
// per-pixel math takes the Gaussian's fields as scalar operands).
__device__ __forceinline__ Splat broadcast(const LaneSplat& l, int j) {
  Splat s;
  s.u = bcast(l.u, j);
  s.v = bcast(l.v, j);
  s.o = bcast(l.o, j);
  s.pa = bcast(l.pa, j);
  s.pb = bcast(l.pb, j);
  s.pc = bcast(l.pc, j);
  s.cut = bcast(l.cut, j);
  s.r = bcast(l.r, j);
  s.g = bcast(l.g, j);
  s.bl = bcast(l.b, j);
  return s;
}

// DPP read of another lane's value (all rows and banks enabled; a lane whose
// source is out of range reads 0).  Combined with an add it compiles to a single
// v_add_f32_dpp.
template <int CTRL>
__device__ __forceinline__ float dpp0(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sum over the 64 lanes, valid in lane 63 only: quad_perm xor 1 and xor 2, row
// half-mirror and mirror (each row of 16 then holds its row sum), row_bcast:15
// (row 3 += row 2, row 1 += row 0) and row_bcast:31 (rows 2, 3 += lane 31).
// Other lanes end with partial sums.  Needs a full EXEC.
__device__ __forceinline__ float wave_sum_lane63(float v) {
  v += dpp0<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp0<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp0<0x141>(v);  // row_half_mirror
  v += dpp0<0x140>(v);  // row_mirror
  v += dpp0<0x142>(v);  // row_bcast:15
  v += dpp0<0x143>(v);  // row_bcast:31
  return v;
}

}  // namespace gs
