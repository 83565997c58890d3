// Projection backward: chain rule from dL/d(u, v, inverse covariance, rgb,
// opacity) to the parameters (mean, quaternion, log-scale, opacity logit, SH
// coefficients), one thread per Gaussian.
//
// Differentiates the forward of project_fwd.hip, i.e. the functions of
// splats/camera.py:81-124, splats/utils.py:8-75 and torch.py:165-203, as torch
// autograd would: clamp/clamp_min pass the gradient on the closed interval,
// F.normalize is differentiated through its norm, and the depth clamp of
// camera.py:97 stops the gradient when |depth| < 1e-4.  Gaussians with
// count == 0 receive zero gradients (project_bwd.py:32,324-334).
// Replaces kernels/rasterize/project_bwd.py:8-381.
#include <algorithm>
#include <cmath>

#include "common.h"
#include "sh.h"

namespace gs {
namespace {

constexpr int kBlock = 256;

// World -> camera extrinsics and the intrinsics the backward needs, by value.
struct BwdCamera {
  float r[9];
  float t[3];
  float fx, fy, lim_x, lim_y;  // lim: 1.3 x tan(half field of view), camera.py:106-116
};

constexpr int kMaxBwdViews = 16;  // views per launch of the multi-view kernel

struct ProjectBwdArgs {
  const float* mean;
  const float* rotation;
  const float* scale;
  const float* opacity;
  const float* color;
  BwdCamera cam[kMaxBwdViews];
  int views;             // cameras in cam[]; view v's inputs are at v * view_stride Gaussians
  int64_t view_stride;   // Gaussians between consecutive views' inputs (n for one view)
  bool accumulate;       // add to the gradient buffers instead of overwriting them
  const float* grad_in;  // [views, N, 9]
  const int32_t* counts;  // [views, N]
  int64_t n;
  float eps;
  float* g_mean;
  float* g_rot;
  float* g_scale;
  float* g_opacity;
  float* g_color;
};

// Gradients of one view's projection of Gaussian gi, added to the
// accumulators: the mean, the quaternion before normalisation (h, turned
// into the raw quaternion's gradient once all views are in), the log-scales,
// the opacity logit and the SH coefficients.
template <int K>
__device__ __forceinline__ void view_gradients(
    const ProjectBwdArgs& a, const BwdCamera& cam, int64_t gi, int64_t vi, float mx, float myy,
    float mz, const double (&q)[4], const double (&sd)[3], float alpha0,
    const float (&coef)[3 * K], float& gmx, float& gmy, float& gmz, float (&h)[4],
    float (&gs3)[3], float& gop, float (&gcoef)[3 * K], const float (&gin)[9]) {
  const float r00 = cam.r[0], r01 = cam.r[1], r02 = cam.r[2];
  const float r10 = cam.r[3], r11 = cam.r[4], r12 = cam.r[5];
  const float r20 = cam.r[6], r21 = cam.r[7], r22 = cam.r[8];
  const float t0 = cam.t[0], t1 = cam.t[1], t2 = cam.t[2];
  const float gu = gin[0], gv = gin[1], gA = gin[2], gB = gin[3], gC = gin[4];
  const float gcol[3] = {gin[5], gin[6], gin[7]};
  const float gal = gin[8];

  // ---- SH colour ----
  const float ex = -(r00 * t0 + r10 * t1 + r20 * t2) - mx;
  const float ey = -(r01 * t0 + r11 * t1 + r21 * t2) - myy;
  const float ez = -(r02 * t0 + r12 * t1 + r22 * t2) - mz;
  const float enorm = sqrtf(ex * ex + ey * ey + ez * ez);
  const float en = fmaxf(enorm, 1e-12f);
  const float dx = ex / en, dy = ey / en, dz = ez / en;
  float basis[K];
  sh::basis<K>(dx, dy, dz, basis);
  float gbasis[K];
  float gc[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k) acc += basis[k] * coef[k * 3 + c];
    // clamp_min(0) passes the gradient where acc + 0.5 >= 0.
    gc[c] = (acc + 0.5f >= 0.0f) ? gcol[c] : 0.0f;
  }
#pragma unroll
  for (int k = 0; k < K; ++k) {
    gbasis[k] = gc[0] * coef[k * 3 + 0] + gc[1] * coef[k * 3 + 1] + gc[2] * coef[k * 3 + 2];
  }
#pragma unroll
  for (int k = 0; k < K; ++k) {
    gcoef[k * 3 + 0] += gc[0] * basis[k];
    gcoef[k * 3 + 1] += gc[1] * basis[k];
    gcoef[k * 3 + 2] += gc[2] * basis[k];
  }
  if (K > 1) {
    float gdx, gdy, gdz;
    sh::basis_vjp<K>(dx, dy, dz, gbasis, gdx, gdy, gdz);
    // Through e / max(|e|, 1e-12); e = camera centre - mean.
    float gex, gey, gez;
    if (enorm > 1e-12f) {
      const float dot = dx * gdx + dy * gdy + dz * gdz;
      gex = (gdx - dx * dot) / enorm;
      gey = (gdy - dy * dot) / enorm;
      gez = (gdz - dz * dot) / enorm;
    } else {
      gex = gdx / 1e-12f;
      gey = gdy / 1e-12f;
      gez = gdz / 1e-12f;
    }
    gmx -= gex;
    gmy -= gey;
    gmz -= gez;
  }

  // ---- opacity: alpha0 = sigmoid(o) ----
  gop += gal * alpha0 * (1.0f - alpha0);

  // ---- the covariance chain, in double precision ----
  // The chain from the parameters through the 2-D covariance and its inverse
  // (J, W = J Rc, N = W Rq, M = N diag(s), Sigma = M M^T + eps I, inv) and
  // back (dL/dSigma = -inv G inv, dL/dM, dL/dRq = W^T dN, the quaternion and
  // Jacobian terms) is recomputed here in double from the parameters rather
  // than taken from the forward's float32 inverse.  For a nearly degenerate
  // Sigma (an edge-on flat splat, a needle) dL/dSigma and dL/dRq are up to
  // ~1e4 times smaller than the products that form them, so in float32 every
  // rounding on the way -- including the stored inverse's -- reaches the scale
  // and rotation gradients amplified by that much (measured: percent-level
  // errors on config 5's flat splats, 1e-4 on config 3's needles).  The chain
  // is a few hundred fp64 operations per (Gaussian, view), a few microseconds
  // per million Gaussians in a kernel bound by its memory traffic.
  const double dr00 = r00, dr01 = r01, dr02 = r02, dr10 = r10, dr11 = r11, dr12 = r12;
  const double dr20 = r20, dr21 = r21, dr22 = r22;
  const double dmx = mx, dmy = myy, dmz = mz;
  const double px = dr00 * dmx + dr01 * dmy + dr02 * dmz + double(t0);
  const double py = dr10 * dmx + dr11 * dmy + dr12 * dmz + double(t1);
  const double pz = dr20 * dmx + dr21 * dmy + dr22 * dmz + double(t2);
  const double d = -pz;
  const bool depth_free = fabs(d) >= 1e-4;
  const double dc = depth_free ? d : copysign(1e-4, d);
  const double rx = px / dc, ry = py / dc;
  const double lim_x = cam.lim_x, lim_y = cam.lim_y;
  const bool in_x = rx >= -lim_x && rx <= lim_x;
  const bool in_y = ry >= -lim_y && ry <= lim_y;
  const double nx = fmin(fmax(rx, -lim_x), lim_x);
  const double ny = fmin(fmax(ry, -lim_y), lim_y);
  const double fxd = cam.fx, fyd = cam.fy;
  const double j00 = fxd / dc, j02 = fxd * nx / dc;
  const double j11 = -fyd / dc, j12 = -fyd * ny / dc;
  const double w0[3] = {j00 * dr00 + j02 * dr20, j00 * dr01 + j02 * dr21, j00 * dr02 + j02 * dr22};
  const double w1[3] = {j11 * dr10 + j12 * dr20, j11 * dr11 + j12 * dr21, j11 * dr12 + j12 * dr22};
  const double qw = q[0], qx = q[1], qy = q[2], qz = q[3];
  const double R[3][3] = {
      {1.0 - 2.0 * (qy * qy + qz * qz), 2.0 * (qx * qy - qw * qz), 2.0 * (qx * qz + qw * qy)},
      {2.0 * (qx * qy + qw * qz), 1.0 - 2.0 * (qx * qx + qz * qz), 2.0 * (qy * qz - qw * qx)},
      {2.0 * (qx * qz - qw * qy), 2.0 * (qy * qz + qw * qx), 1.0 - 2.0 * (qx * qx + qy * qy)}};
  // N = W Rq (2x3), M = N diag(s).
  double N[2][3], M[2][3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    N[0][c] = w0[0] * R[0][c] + w0[1] * R[1][c] + w0[2] * R[2][c];
    N[1][c] = w1[0] * R[0][c] + w1[1] * R[1][c] + w1[2] * R[2][c];
    M[0][c] = N[0][c] * sd[c];
    M[1][c] = N[1][c] * sd[c];
  }
  const double eps = a.eps;
  const double c00 = M[0][0] * M[0][0] + M[0][1] * M[0][1] + M[0][2] * M[0][2] + eps;
  const double c01 = M[0][0] * M[1][0] + M[0][1] * M[1][1] + M[0][2] * M[1][2];
  const double c11 = M[1][0] * M[1][0] + M[1][1] * M[1][1] + M[1][2] * M[1][2] + eps;
  const double rdet = 1.0 / (c00 * c11 - c01 * c01);
  const double i00 = c11 * rdet, i01 = -c01 * rdet, i11 = c00 * rdet;

  // ---- through the 2x2 inverse: dL/dSigma = -inv G inv ----
  const double dA = gA, dB = gB, dC = gC;
  const double t00 = i00 * dA + i01 * dB, t01 = i00 * dB + i01 * dC;
  const double t10 = i01 * dA + i11 * dB, t11 = i01 * dB + i11 * dC;
  const double k00 = -(t00 * i00 + t01 * i01);
  const double k01 = -(t00 * i01 + t01 * i11);
  const double k11 = -(t10 * i01 + t11 * i11);

  // ---- Sigma = M M^T + eps I: dL/dM = 2 K M ----
  double dN[2][3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const double dm0 = 2.0 * (k00 * M[0][c] + k01 * M[1][c]);
    const double dm1 = 2.0 * (k01 * M[0][c] + k11 * M[1][c]);
    dN[0][c] = dm0 * sd[c];
    dN[1][c] = dm1 * sd[c];
    gs3[c] += float((dm0 * N[0][c] + dm1 * N[1][c]) * sd[c]);  // d/dlog s = d/ds * s
  }
  // dRq = W^T dN; dW = dN Rq^T.
  double G[3][3];
#pragma unroll
  for (int r = 0; r < 3; ++r)
#pragma unroll
    for (int c = 0; c < 3; ++c) G[r][c] = w0[r] * dN[0][c] + w1[r] * dN[1][c];
  double dW0[3], dW1[3];
#pragma unroll
  for (int kk = 0; kk < 3; ++kk) {
    dW0[kk] = dN[0][0] * R[kk][0] + dN[0][1] * R[kk][1] + dN[0][2] * R[kk][2];
    dW1[kk] = dN[1][0] * R[kk][0] + dN[1][1] * R[kk][1] + dN[1][2] * R[kk][2];
  }

  // ---- rotation matrix -> normalised quaternion (this view's term rounded once) ----
  h[0] += float(2.0 * (qz * (G[1][0] - G[0][1]) + qy * (G[0][2] - G[2][0]) + qx * (G[2][1] - G[1][2])));
  h[1] += float(2.0 * (qy * (G[0][1] + G[1][0]) + qz * (G[0][2] + G[2][0]) + qw * (G[2][1] - G[1][2])) -
                4.0 * qx * (G[1][1] + G[2][2]));
  h[2] += float(2.0 * (qx * (G[0][1] + G[1][0]) + qw * (G[0][2] - G[2][0]) + qz * (G[1][2] + G[2][1])) -
                4.0 * qy * (G[0][0] + G[2][2]));
  h[3] += float(2.0 * (qw * (G[1][0] - G[0][1]) + qx * (G[0][2] + G[2][0]) + qy * (G[1][2] + G[2][1])) -
                4.0 * qz * (G[0][0] + G[1][1]));

  // ---- W = J Rc: dJ entries ----
  const double dj00 = dW0[0] * dr00 + dW0[1] * dr01 + dW0[2] * dr02;
  const double dj02 = dW0[0] * dr20 + dW0[1] * dr21 + dW0[2] * dr22;
  const double dj11 = dW1[0] * dr10 + dW1[1] * dr11 + dW1[2] * dr12;
  const double dj12 = dW1[0] * dr20 + dW1[1] * dr21 + dW1[2] * dr22;

  // ---- camera-space point ----
  // u = fx x / d + cx and v = -fy y / d + cy use the unclamped depth.
  const double d2 = d * d;
  double gpx = gu * fxd / d;
  double gpy = -gv * fyd / d;
  double gd = -gu * fxd * px / d2 + gv * fyd * py / d2;
  // Jacobian terms use the clamped depth dc.
  const double dc2 = dc * dc, dc3 = dc2 * dc;
  if (in_x) gpx += dj02 * fxd / dc2;
  if (in_y) gpy += dj12 * (-fyd / dc2);
  if (depth_free) {
    double gdc = -dj00 * fxd / dc2 + dj11 * fyd / dc2;
    gdc += dj02 * (-fxd * nx / dc2 - (in_x ? fxd * px / dc3 : 0.0));
    gdc += dj12 * (fyd * ny / dc2 + (in_y ? fyd * py / dc3 : 0.0));
    gd += gdc;
  }
  const double gpz = -gd;
  gmx += float(dr00 * gpx + dr10 * gpy + dr20 * gpz);
  gmy += float(dr01 * gpx + dr11 * gpy + dr21 * gpz);
  gmz += float(dr02 * gpx + dr12 * gpy + dr22 * gpz);

}

// MULTI = false: one view, no accumulation (the single-camera entry point),
// which lets the compiler drop the view loop and keep fewer values live.
// The block's SH coefficients come in through LDS with coalesced 16-byte loads
// and their gradients leave the same way (sh::stage_block / unstage_block);
// each thread keeps its own Gaussian's coefficients and gradients in
// registers in between.
template <int K, bool MULTI>
__global__ __launch_bounds__(kBlock) void project_bwd_kernel(ProjectBwdArgs a) {
  constexpr int F = 3 * K;
  constexpr int S = sh::row_stride<F>();
  __shared__ __align__(16) float coeff[kBlock * S];
  const int views = MULTI ? a.views : 1;
  const bool accumulate = MULTI && a.accumulate;
  const int64_t base = int64_t(blockIdx.x) * kBlock;
  const int nvalid = int(min(int64_t(kBlock), a.n - base));
  const int64_t gi = base + threadIdx.x;
  const bool have = gi < a.n;
  // The Gaussian's own parameters and count are requested before the block's
  // coefficients, so all of these loads are in flight together (threads past
  // the end read the last Gaussian and write nothing).
  const int64_t gl = have ? gi : a.n - 1;
  const float mx = load_nt(a.mean + gl * 3 + 0), myy = load_nt(a.mean + gl * 3 + 1),
              mz = load_nt(a.mean + gl * 3 + 2);
  const float lop = load_nt(a.opacity + gl);
  const float4 qr = load_nt(reinterpret_cast<const float4*>(a.rotation) + gl);
  const float ls0 = load_nt(a.scale + gl * 3 + 0), ls1 = load_nt(a.scale + gl * 3 + 1),
              ls2 = load_nt(a.scale + gl * 3 + 2);
  const int32_t count0 = load_nt(a.counts + gl);
  // One view: its gradient inputs too.
  float gin0[9];
  if (!MULTI) {
#pragma unroll
    for (int i = 0; i < 9; ++i) gin0[i] = load_nt(a.grad_in + gl * 9 + i);
  }
  sh::stage_block<F, kBlock>(a.color + base * F, nvalid, coeff);
  __syncthreads();
  float gmx = 0.0f, gmy = 0.0f, gmz = 0.0f;
  float h[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float gs3[3] = {0.0f, 0.0f, 0.0f};
  float gop = 0.0f;
  float gcoef[F];
#pragma unroll
  for (int i = 0; i < F; ++i) gcoef[i] = 0.0f;
  bool any = have && count0 != 0;
  for (int v = 1; have && v < views; ++v) any |= a.counts[v * a.view_stride + gi] != 0;
  double q[4] = {0.0, 0.0, 0.0, 0.0};
  double qnorm = 0.0;
  if (any) {
    // Parameters are read once, only for Gaussians some view counted.
    float coef[F];
    sh::row_load<F>(coeff, threadIdx.x, coef);
    const float alpha0 = 1.0f / (1.0f + expf(-lop));
    // The normalised quaternion and the scales in double (see view_gradients).
    qnorm = sqrt(double(qr.x) * qr.x + double(qr.y) * qr.y + double(qr.z) * qr.z +
                 double(qr.w) * qr.w);
    const double qn = fmax(qnorm, 1e-12);
    q[0] = qr.x / qn;
    q[1] = qr.y / qn;
    q[2] = qr.z / qn;
    q[3] = qr.w / qn;
    const double sd[3] = {exp(double(ls0)), exp(double(ls1)), exp(double(ls2))};
    if (!MULTI) {  // count0 != 0 here
      view_gradients<K>(a, a.cam[0], gi, gi, mx, myy, mz, q, sd, alpha0, coef, gmx, gmy, gmz, h,
                        gs3, gop, gcoef, gin0);
    } else {
      for (int v = 0; v < views; ++v) {
        const int64_t vi = v * a.view_stride + gi;
        if (a.counts[vi] == 0) continue;  // zero gradient from this view (project_bwd.py:324-334)
        float gin[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) gin[i] = a.grad_in[vi * 9 + i];
        view_gradients<K>(a, a.cam[v], gi, vi, mx, myy, mz, q, sd, alpha0, coef, gmx, gmy, gmz,
                          h, gs3, gop, gcoef, gin);
      }
    }
  }
  // ---- normalised quaternion -> raw quaternion (linear in h, so once) ----
  float gq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (any) {
    if (qnorm > 1e-12) {
      // The normalisation's Jacobian removes h's radial part, which can be
      // much larger than the result: formed in double.
      const double dot = q[0] * h[0] + q[1] * h[1] + q[2] * h[2] + q[3] * h[3];
#pragma unroll
      for (int i = 0; i < 4; ++i) gq[i] = float((h[i] - q[i] * dot) / qnorm);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) gq[i] = h[i] / 1e-12f;
    }
  }
  if (have && accumulate) {
    gmx += a.g_mean[gi * 3 + 0];
    gmy += a.g_mean[gi * 3 + 1];
    gmz += a.g_mean[gi * 3 + 2];
    const float4 r = reinterpret_cast<const float4*>(a.g_rot)[gi];
    gq[0] += r.x;
    gq[1] += r.y;
    gq[2] += r.z;
    gq[3] += r.w;
#pragma unroll
    for (int c = 0; c < 3; ++c) gs3[c] += a.g_scale[gi * 3 + c];
    gop += a.g_opacity[gi];
    float prev[F];
    sh::load_coefficients<K>(a.g_color + gi * F, prev);
#pragma unroll
    for (int i = 0; i < F; ++i) gcoef[i] += prev[i];
  }
  if (have) {
    store_nt(gmx, a.g_mean + gi * 3 + 0);
    store_nt(gmy, a.g_mean + gi * 3 + 1);
    store_nt(gmz, a.g_mean + gi * 3 + 2);
    store_nt(make_float4(gq[0], gq[1], gq[2], gq[3]), reinterpret_cast<float4*>(a.g_rot) + gi);
    store_nt(gs3[0], a.g_scale + gi * 3 + 0);
    store_nt(gs3[1], a.g_scale + gi * 3 + 1);
    store_nt(gs3[2], a.g_scale + gi * 3 + 2);
    store_nt(gop, a.g_opacity + gi);
    // Each thread overwrites only its own row, which only it has read.
    sh::row_store<F>(coeff, threadIdx.x, gcoef);
  }
  __syncthreads();
  sh::unstage_block<F, kBlock>(a.g_color + base * F, nvalid, coeff);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace gs

using namespace gs;

namespace {

// Chain rule for `views` cameras (host arrays as for the forward), summing
// every view's gradient per Gaussian; launches of up to kMaxBwdViews views,
// the later ones adding to the earlier ones' results.
int project_bwd_views(const float* mean, const float* rotation, const float* scale,
                      const float* opacity, const float* color, int64_t n, int32_t num_sh,
                      const float* camera_rotations, const float* camera_translations,
                      const float* intrinsics, int views, gs_view view,
                      const float* /*inverse_covariance*/, const float* grad_projected,
                      const int32_t* counts, float* grad_mean, float* grad_rotation,
                      float* grad_scale, float* grad_opacity, float* grad_color, void* stream) {
  GS_REQUIRE(n >= 0, GS_ERR_INVALID_ARGUMENT, "negative Gaussian count");
  GS_REQUIRE(num_sh == 1 || num_sh == 4 || num_sh == 9 || num_sh == 16, GS_ERR_UNSUPPORTED,
             "SH degrees above 3 are not implemented (got %d coefficients)", num_sh);
  if (n == 0) return GS_OK;
  GS_REQUIRE(mean && rotation && scale && opacity && color && camera_rotations &&
                 camera_translations && grad_projected && counts &&
                 grad_mean && grad_rotation && grad_scale && grad_opacity && grad_color,
             GS_ERR_INVALID_ARGUMENT, "null pointer argument");
  GS_REQUIRE(aligned16(rotation) && aligned16(color) && aligned16(grad_rotation) &&
                 aligned16(grad_color),
             GS_ERR_INVALID_ARGUMENT, "rotation/color buffers must be 16-byte aligned");
  GS_REQUIRE(int64_t(views) * n < (int64_t(1) << 31), GS_ERR_OVERFLOW,
             "too many Gaussians (%lld x %d views)", (long long)n, views);
  ProjectBwdArgs a;
  a.mean = mean;
  a.rotation = rotation;
  a.scale = scale;
  a.opacity = opacity;
  a.color = color;
  a.view_stride = n;
  a.n = n;
  a.eps = view.covariance_epsilon;
  a.g_mean = grad_mean;
  a.g_rot = grad_rotation;
  a.g_scale = grad_scale;
  a.g_opacity = grad_opacity;
  a.g_color = grad_color;
  const dim3 grid(unsigned(ceil_div(n, kBlock)));
  hipStream_t s = as_stream(stream);
  for (int first = 0; first < views; first += kMaxBwdViews) {
    a.views = std::min(kMaxBwdViews, views - first);
    for (int j = 0; j < a.views; ++j) {
      const int vw = first + j;
      BwdCamera& c = a.cam[j];
      // Host memory: the cameras travel as kernel arguments.
      for (int i = 0; i < 9; ++i) c.r[i] = camera_rotations[vw * 9 + i];
      for (int i = 0; i < 3; ++i) c.t[i] = camera_translations[vw * 3 + i];
      c.fx = intrinsics ? intrinsics[vw * 4 + 0] : view.fx;
      c.fy = intrinsics ? intrinsics[vw * 4 + 1] : view.fy;
      GS_REQUIRE(c.fx != 0.0f && c.fy != 0.0f, GS_ERR_INVALID_ARGUMENT,
                 "zero focal length (view %d)", vw);
      c.lim_x = float(1.3 * (double(view.image_width) / (2.0 * double(c.fx))));
      c.lim_y = float(1.3 * (double(view.image_height) / (2.0 * double(c.fy))));
    }
    const int64_t off = int64_t(first) * n;
    a.grad_in = grad_projected + off * 9;
    a.counts = counts + off;
    a.accumulate = first > 0;
    if (views == 1) {
      switch (num_sh) {
        case 1: launch_timed(project_bwd_kernel<1, false>, grid, kBlock, 0, s, a); break;
        case 4: launch_timed(project_bwd_kernel<4, false>, grid, kBlock, 0, s, a); break;
        case 9: launch_timed(project_bwd_kernel<9, false>, grid, kBlock, 0, s, a); break;
        default: launch_timed(project_bwd_kernel<16, false>, grid, kBlock, 0, s, a); break;
      }
    } else {
      switch (num_sh) {
        case 1: launch_timed(project_bwd_kernel<1, true>, grid, kBlock, 0, s, a); break;
        case 4: launch_timed(project_bwd_kernel<4, true>, grid, kBlock, 0, s, a); break;
        case 9: launch_timed(project_bwd_kernel<9, true>, grid, kBlock, 0, s, a); break;
        default: launch_timed(project_bwd_kernel<16, true>, grid, kBlock, 0, s, a); break;
      }
    }
    GS_TRY(check_launch("project_bwd"));
  }
  return GS_OK;
}

}  // namespace

extern "C" GS_API int gs_project_bwd(const float* mean, const float* rotation, const float* scale,
                                     const float* opacity, const float* color, int64_t n,
                                     int32_t num_sh, const float* camera_rotation,
                                     const float* camera_translation, gs_view view,
                                     const float* inverse_covariance,
                                     const float* grad_projected, const int32_t* counts,
                                     float* grad_mean, float* grad_rotation, float* grad_scale,
                                     float* grad_opacity, float* grad_color, void* stream) {
  clear_error();
  return project_bwd_views(mean, rotation, scale, opacity, color, n, num_sh, camera_rotation,
                           camera_translation, nullptr, 1, view, inverse_covariance,
                           grad_projected, counts, grad_mean, grad_rotation, grad_scale,
                           grad_opacity, grad_color, stream);
}

extern "C" GS_API int gs_project_bwd_views(
    const float* mean, const float* rotation, const float* scale, const float* opacity,
    const float* color, int64_t n, int32_t num_sh, const float* camera_rotations,
    const float* camera_translations, const float* intrinsics, gs_view view,
    const float* inverse_covariance, const float* grad_projected, const int32_t* counts,
    float* grad_mean, float* grad_rotation, float* grad_scale, float* grad_opacity,
    float* grad_color, void* stream) {
  clear_error();
  return project_bwd_views(mean, rotation, scale, opacity, color, n, num_sh, camera_rotations,
                           camera_translations, intrinsics, mosaic_of(view).views, view,
                           inverse_covariance, grad_projected, counts, grad_mean, grad_rotation,
                           grad_scale, grad_opacity, grad_color, stream);
}
