// Per-pixel compositing math shared by the forward and backward kernels, so both
// evaluate bit-identical alphas.
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace gs {

constexpr float kMinAlpha = 1.0f / 255.0f;  // torch.py:350, composite.py:82
constexpr float kMaxAlpha = 0.99f;          // torch.py:349, composite.py:81
constexpr float kNegHalfLog2e = -0.72134752044448170f;  // -0.5 / ln 2

// Gaussian broadcast to every lane of a wave (values live in SGPRs).
struct Splat {
  float u, v, o, a, b, c, cut, r, g, bl;
};

// Quadratic form of the inverse covariance at pixel offset (dx, dy), in the
// term order of utils.py:78-87 / composite.py:73.
__device__ __forceinline__ float quad_form(const Splat& s, float dx, float dy) {
  return s.a * dx * dx + 2.0f * s.b * dx * dy + s.c * dy * dy;
}

// Unclamped alpha = opacity * probability (utils.py:90-99); `prob` returns the
// probability.  Gaussian mode uses exp(-D/2) = exp2(-D/(2 ln 2)).
template <bool ELLIPSOID>
__device__ __forceinline__ float raw_alpha(const Splat& s, float D, float& prob) {
  if constexpr (ELLIPSOID) {
    prob = D <= s.cut ? 1.0f : 0.0f;
  } else {
    prob = __builtin_amdgcn_exp2f(D * kNegHalfLog2e);
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

__device__ __forceinline__ float bcast(float x, int j) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j));
}

// Broadcasts lane j's record to the whole wave (v_readlane into SGPRs, so the
// per-pixel math takes the Gaussian's fields as scalar operands).
__device__ __forceinline__ Splat broadcast(const GsRecord& r, int j) {
  Splat s;
  s.u = bcast(r.u, j);
  s.v = bcast(r.v, j);
  s.o = bcast(r.opacity, j);
  s.a = bcast(r.inv00, j);
  s.b = bcast(r.inv01, j);
  s.c = bcast(r.inv11, j);
  s.cut = bcast(r.cut, j);
  s.r = bcast(r.r, j);
  s.g = bcast(r.g, j);
  s.bl = bcast(r.b, j);
  return s;
}

}  // namespace gs
