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
  float oa, ob, oc;  // opacity times the unscaled inverse covariance (mean gradient)
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
  s.oa = r.opacity * r.inv00;
  s.ob = r.opacity * r.inv01;
  s.oc = r.opacity * r.inv11;
  return s;
}

// A lane owns one pixel column of its tile (pixel q = lane + 64 k lies in
// column lane % tile for every tile size up to 64), so the part of the
// exponent that depends only on dx is computed once per (lane, splat):
//   log2 falloff = pa dx^2 + pb dx dy + pc dy^2 = p0 + dy (p1 + pc dy).
// The forward and backward kernels both evaluate it through these helpers, so
// their alphas are bit-identical.
struct ColumnTerms {
  float dx, p0, p1;
};

__device__ __forceinline__ ColumnTerms column_terms(const Splat& s, float px) {
  ColumnTerms c;
  c.dx = px - s.u;
  c.p1 = s.pb * c.dx;
  c.p0 = (s.pa * c.dx) * c.dx;
  return c;
}

__device__ __forceinline__ float falloff_log2(const ColumnTerms& c, float pc, float dy) {
  return fmaf(dy, fmaf(pc, dy, c.p1), c.p0);
}

// Unclamped alpha = opacity * probability (utils.py:90-99); `prob` returns the
// probability.  Ellipsoid mode compares D = power / (-0.5 log2 e) with the
// cutoff stored in the record.
template <bool ELLIPSOID>
__device__ __forceinline__ float raw_alpha(const Splat& s, const ColumnTerms& c, float dy,
                                           float& prob) {
  const float power = falloff_log2(c, s.pc, dy);
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
// The vertices use v_rcp_f32 reciprocals: an inexact vertex only raises the
// value found by a second-order amount, far below the margin callers add.
__device__ __forceinline__ float min_quad_over_rect(float a, float b, float c, float u, float v,
                                                    float x0, float x1, float y0, float y1) {
  const float lx = x0 - u, hx = x1 - u, ly = y0 - v, hy = y1 - v;
  if (lx <= 0.0f && hx >= 0.0f && ly <= 0.0f && hy >= 0.0f) return 0.0f;
  if (!(a > 0.0f) || !(c > 0.0f)) return 0.0f;  // degenerate: never skip
  const float nbc = -b * __builtin_amdgcn_rcpf(c), nba = -b * __builtin_amdgcn_rcpf(a);
  float best = 3.0e38f;
  const float ex[2] = {lx, hx};
  const float ey[2] = {ly, hy};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float dx = ex[i];
    const float dy = fminf(fmaxf(nbc * dx, ly), hy);
    best = fminf(best, dx * (a * dx + 2.0f * b * dy) + c * dy * dy);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float dy = ey[i];
    const float dx = fminf(fmaxf(nba * dy, lx), hx);
    best = fminf(best, dx * (a * dx + 2.0f * b * dy) + c * dy * dy);
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

// Columns and rows spanned by the set lanes of a 64-pixel band's ballot `m`
// (m != 0), lane l holding the band's pixel in column l % TILE, row l / TILE:
// `cols` gets bit c for every column with a set lane (the band's rows ORed
// into the low TILE bits), r0 / r1 the first and last row.  Scalar work on a
// wave-uniform mask.
template <int TILE>
__device__ __forceinline__ void band_span(uint64_t m, uint32_t& cols, int& r0, int& r1) {
  uint64_t f = m;
#pragma unroll
  for (int s = 32; s >= TILE; s >>= 1) f |= f >> s;
  cols = uint32_t(f) & uint32_t((uint64_t(1) << TILE) - 1);
  r0 = __builtin_ctzll(m) / TILE;
  r1 = (63 - __builtin_clzll(m)) / TILE;
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

// Sum over each row of 16 lanes, left in every lane of the row: quad_perm
// xor 1 and xor 2, then row half-mirror and row mirror.  Needs a full EXEC.
__device__ __forceinline__ float row_sum(float v) {
  v += dpp0<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp0<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp0<0x141>(v);  // row_half_mirror
  v += dpp0<0x140>(v);  // row_mirror
  return v;
}

// v_permlane32_swap exchanges the upper half of x with the lower half of y, so
// the sum holds x folded over the two halves in lanes 0-31 and y folded in
// lanes 32-63: lane i < 32 gets x[i] + x[i + 32], lane i >= 32 gets
// y[i - 32] + y[i].
__device__ __forceinline__ float fold_halves(float x, float y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// v_permlane16_swap exchanges the odd rows of x with the even rows of y; the
// sum holds rows (x0 + x1, y0 + y1, x2 + x3, y2 + y3).
__device__ __forceinline__ float fold_rows(float x, float y) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Wave totals of nine per-lane values v[0..8] by a transposing reduction:
// the two swap folds spread the values over the rows of three registers and a
// row sum finishes each, 30 VALU operations instead of 54 for nine full
// butterflies.  On return, every lane of row r (lanes 16 r .. 16 r + 15) of
//   t0 holds the total of v[sum9_field(r)],  t1 that of v[4 + sum9_field(r)],
// and t2 holds the total of v[8] in every lane.  Needs a full EXEC.
__device__ __forceinline__ int sum9_field(int row) { return ((row & 1) << 1) | (row >> 1); }

__device__ __forceinline__ void wave_sum9(const float (&v)[9], float& t0, float& t1, float& t2) {
  const float a0 = fold_halves(v[0], v[1]);
  const float a1 = fold_halves(v[2], v[3]);
  const float a2 = fold_halves(v[4], v[5]);
  const float a3 = fold_halves(v[6], v[7]);
  const float a4 = fold_halves(v[8], v[8]);
  t0 = row_sum(fold_rows(a0, a1));  // rows: v0, v2, v1, v3
  t1 = row_sum(fold_rows(a2, a3));  // rows: v4, v6, v5, v7
  t2 = row_sum(fold_rows(a4, a4));  // every row: v8
}

}  // namespace gs
