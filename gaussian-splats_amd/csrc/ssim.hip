// Structural similarity of the training step (training/train.py:139 through
// training/utils.py:65-67, torchmetrics' structural_similarity_index_measure
// with data_range = 1 and its defaults: Gaussian window sigma = 1.5 of
// 2 * int(3.5 sigma + 0.5) + 1 = 11 taps normalised to sum 1, k1 = 0.01,
// k2 = 0.03, variances clamped at 0, the map cropped by the window radius on
// every side (where the window never reaches the padding), mean over pixels
// and channels).
//
// Per channel, with w the window and x, y the image and target:
//   mx = w*x, my = w*y, sxx = w*x^2 - mx^2 (>= 0), syy = w*y^2 - my^2 (>= 0),
//   sxy = w*xy - mx my,  A = 2 mx my + c1,  B = 2 sxy + c2,
//   C = mx^2 + my^2 + c1,  D = sxx + syy + c2,  s = A B / (C D).
// Gradient with respect to x of the mean S = sum(s) / M:
//   dS/dx(q) = (1/M) [ (w * Gm)(q) + 2 x(q) (w * Gxx)(q) + y(q) (w * Gxy)(q) ]
// with, per pixel of the cropped map (zero elsewhere),
//   Gm  = 2 my (B - A) / (C D) - 2 mx s / C + 2 mx s [sxx clamp passes] / D,
//   Gxx = -s [sxx clamp passes] / D,   Gxy = 2 A / (C D)
// (w is symmetric, so correlation and convolution agree).  The forward writes
// Gm, Gxx, Gxy; the backward filters them.
//
// Layout: image, target and gradient [H, W, 3] (channels innermost, as the
// rasterizer writes them); the three G maps [3, H, W, 3].  Each workgroup
// covers a 32 x 16 block of output pixels: the block plus the window radius
// is staged through LDS, filtered along rows, then along columns.
#include <algorithm>
#include <cmath>

#include "common.h"

namespace gs {
namespace {

constexpr int kR = 5;                  // window radius
constexpr int kTaps = 2 * kR + 1;      // 11
constexpr int kBW = 32, kBH = 16;      // output block
constexpr int kInW = kBW + 2 * kR;     // 42
constexpr int kInH = kBH + 2 * kR;     // 26
constexpr int kSsimThreads = 256;
constexpr int kStagePer = (kInH * kInW + kSsimThreads - 1) / kSsimThreads;  // staged pixels per thread
constexpr int kSsimPartials = 65536;   // forward workgroups at most (one partial sum each)

struct SsimWeights {
  float w[kTaps];
};

// Forward: the cropped SSIM map's partial sums and the three G maps.
__global__ __launch_bounds__(kSsimThreads) void ssim_fwd_kernel(
    const float* __restrict__ x, const float* __restrict__ y, int H, int W, SsimWeights wt,
    float c1, float c2, float* __restrict__ gmap, float* __restrict__ partial) {
  __shared__ float in_x[kInH][kInW + 1];
  __shared__ float in_y[kInH][kInW + 1];
  __shared__ float rows[5][kInH][kBW + 1];
  __shared__ float red[kSsimThreads / 64];
  const int bx = blockIdx.x * kBW + kR, by = blockIdx.y * kBH + kR;  // first output pixel
  const int64_t plane = int64_t(H) * W * 3;
  // The block's staged pixels of all three channels are requested at once
  // (coordinates clamped into the image, values outside replaced by 0), so
  // the loads are in flight together instead of one round trip per element.
  float vx[3][kStagePer], vy[3][kStagePer];
#pragma unroll
  for (int k = 0; k < kStagePer; ++k) {
    const int i = threadIdx.x + k * kSsimThreads;
    const int r = i / kInW, q = i - r * kInW;
    const int gy = by - kR + r, gx = bx - kR + q;
    const bool in = i < kInH * kInW && gy < H && gx < W;  // gy, gx >= 0 by construction
    const int64_t o = (int64_t(min(gy, H - 1)) * W + min(gx, W - 1)) * 3;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      vx[c][k] = x[o + c];
      vy[c][k] = y[o + c];
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      if (!in) vx[c][k] = vy[c][k] = 0.0f;
    }
  }
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    __syncthreads();  // the previous channel's LDS reads are done
#pragma unroll
    for (int k = 0; k < kStagePer; ++k) {
      const int i = threadIdx.x + k * kSsimThreads;
      if (i < kInH * kInW) {
        const int r = i / kInW, q = i - r * kInW;
        in_x[r][q] = vx[c][k];
        in_y[r][q] = vy[c][k];
      }
    }
    __syncthreads();
    // Row pass: the five moments filtered along x for every staged row.
    for (int i = threadIdx.x; i < kInH * kBW; i += kSsimThreads) {
      const int r = i / kBW, q = i - r * kBW;
      float m[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int t = 0; t < kTaps; ++t) {
        const float a = in_x[r][q + t], b = in_y[r][q + t], w = wt.w[t];
        m[0] += w * a;
        m[1] += w * b;
        m[2] += w * (a * a);
        m[3] += w * (b * b);
        m[4] += w * (a * b);
      }
#pragma unroll
      for (int k = 0; k < 5; ++k) rows[k][r][q] = m[k];
    }
    __syncthreads();
    // Column pass and the SSIM terms of the block's output pixels.
    for (int i = threadIdx.x; i < kBH * kBW; i += kSsimThreads) {
      const int r = i / kBW, q = i - r * kBW;
      const int gy = by + r, gx = bx + q;
      if (gy >= H - kR || gx >= W - kR) continue;
      float m[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int t = 0; t < kTaps; ++t) {
        const float w = wt.w[t];
#pragma unroll
        for (int k = 0; k < 5; ++k) m[k] += w * rows[k][r + t][q];
      }
      const float mx = m[0], my = m[1];
      const float vxx = m[2] - mx * mx, vyy = m[3] - my * my;
      const bool pass_x = vxx >= 0.0f;
      const float sxx = fmaxf(vxx, 0.0f), syy = fmaxf(vyy, 0.0f);
      const float sxy = m[4] - mx * my;
      const float A = 2.0f * mx * my + c1, B = 2.0f * sxy + c2;
      const float C = mx * mx + my * my + c1, D = sxx + syy + c2;
      const float inv = 1.0f / (C * D);
      const float s = A * B * inv;
      acc += s;
      const float gm = 2.0f * my * (B - A) * inv - 2.0f * mx * s / C +
                       (pass_x ? 2.0f * mx * s / D : 0.0f);
      const float gxx = pass_x ? -s / D : 0.0f;
      const float gxy = 2.0f * A * inv;
      const int64_t o = (int64_t(gy) * W + gx) * 3 + c;
      gmap[o] = gm;
      gmap[plane + o] = gxx;
      gmap[2 * plane + o] = gxy;
    }
  }
  // Workgroup sum in a fixed order.
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.0f;
    for (int i = 0; i < kSsimThreads / 64; ++i) s += red[i];
    partial[blockIdx.y * gridDim.x + blockIdx.x] = s;
  }
}

__global__ __launch_bounds__(kSsimThreads) void ssim_finish_kernel(const float* __restrict__ partial,
                                                                   int blocks, double count,
                                                                   float* __restrict__ out) {
  __shared__ double red[kSsimThreads / 64];
  double acc = 0.0;
  for (int i = threadIdx.x; i < blocks; i += kSsimThreads) acc += double(partial[i]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int i = 0; i < kSsimThreads / 64; ++i) s += red[i];
    out[0] = float(s / count);
  }
}

// Backward: grad(q) = g / M [ (w*Gm)(q) + 2 x(q) (w*Gxx)(q) + y(q) (w*Gxy)(q) ]
// for every pixel, G = 0 outside the cropped map.  Output blocks tile the
// whole image; the staged window reaches kR beyond the block on each side.
__global__ __launch_bounds__(kSsimThreads) void ssim_bwd_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ gmap,
    const float* __restrict__ grad_out, float inv_count, int H, int W, SsimWeights wt,
    float* __restrict__ grad) {
  __shared__ float in_g[3][kInH][kInW + 1];
  __shared__ float rows[3][kInH][kBW + 1];
  const int bx = blockIdx.x * kBW, by = blockIdx.y * kBH;
  const int64_t plane = int64_t(H) * W * 3;
  const float scale = grad_out[0] * inv_count;
  // As in the forward, all of the thread's loads are issued before the first
  // LDS store: the staged G maps of all channels (coordinates clamped into
  // the cropped map, values outside it replaced by 0) and its output pixels'
  // image and target values.
  float vg[3][3][kStagePer];
#pragma unroll
  for (int k = 0; k < kStagePer; ++k) {
    const int i = threadIdx.x + k * kSsimThreads;
    const int r = i / kInW, q = i - r * kInW;
    const int gy = by - kR + r, gx = bx - kR + q;
    const bool in = i < kInH * kInW && gy >= kR && gy < H - kR && gx >= kR && gx < W - kR;
    const int64_t o = (int64_t(min(max(gy, kR), H - kR - 1)) * W + min(max(gx, kR), W - kR - 1)) * 3;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
#pragma unroll
      for (int m = 0; m < 3; ++m) vg[m][c][k] = gmap[m * plane + o + c];
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
#pragma unroll
      for (int m = 0; m < 3; ++m)
        if (!in) vg[m][c][k] = 0.0f;
    }
  }
  constexpr int kOutPer = kBH * kBW / kSsimThreads;  // output pixels per thread
  float ox[3][kOutPer], oy[3][kOutPer];
#pragma unroll
  for (int k = 0; k < kOutPer; ++k) {
    const int i = threadIdx.x + k * kSsimThreads;
    const int r = i / kBW, q = i - r * kBW;
    const int64_t o = (int64_t(min(by + r, H - 1)) * W + min(bx + q, W - 1)) * 3;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      ox[c][k] = x[o + c];
      oy[c][k] = y[o + c];
    }
  }
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kStagePer; ++k) {
      const int i = threadIdx.x + k * kSsimThreads;
      if (i < kInH * kInW) {
        const int r = i / kInW, q = i - r * kInW;
#pragma unroll
        for (int m = 0; m < 3; ++m) in_g[m][r][q] = vg[m][c][k];
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < kInH * kBW; i += kSsimThreads) {
      const int r = i / kBW, q = i - r * kBW;
      float m[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int t = 0; t < kTaps; ++t) {
        const float w = wt.w[t];
#pragma unroll
        for (int k = 0; k < 3; ++k) m[k] += w * in_g[k][r][q + t];
      }
#pragma unroll
      for (int k = 0; k < 3; ++k) rows[k][r][q] = m[k];
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kOutPer; ++kk) {
      const int i = threadIdx.x + kk * kSsimThreads;
      const int r = i / kBW, q = i - r * kBW;
      const int gy = by + r, gx = bx + q;
      if (gy >= H || gx >= W) continue;
      float m[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int t = 0; t < kTaps; ++t) {
        const float w = wt.w[t];
#pragma unroll
        for (int k = 0; k < 3; ++k) m[k] += w * rows[k][r + t][q];
      }
      const int64_t o = (int64_t(gy) * W + gx) * 3 + c;
      grad[o] = scale * (m[0] + 2.0f * ox[c][kk] * m[1] + oy[c][kk] * m[2]);
    }
  }
}

// torchmetrics' window: exp(-(d / sigma)^2 / 2) for d = -5..5, normalised to
// sum 1, in float32.
SsimWeights window() {
  SsimWeights wt;
  float sum = 0.0f;
  for (int t = 0; t < kTaps; ++t) {
    const float d = float(t - kR) / 1.5f;
    wt.w[t] = std::exp(-(d * d) / 2.0f);
    sum += wt.w[t];
  }
  for (int t = 0; t < kTaps; ++t) wt.w[t] /= sum;
  return wt;
}

dim3 fwd_grid(int H, int W) {
  return dim3(unsigned(ceil_div(W - 2 * kR, kBW)), unsigned(ceil_div(H - 2 * kR, kBH)));
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" {

GS_API size_t gs_ssim_workspace_bytes(int32_t height, int32_t width) {
  if (height <= 2 * kR || width <= 2 * kR) return 0;
  const int64_t maps = 3 * int64_t(height) * width * 3 * int64_t(sizeof(float));
  return align_up(size_t(maps)) + align_up(size_t(kSsimPartials) * sizeof(float));
}

GS_API int gs_ssim_fwd(const float* image, const float* target, int32_t height, int32_t width,
                       float* ssim, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  GS_REQUIRE(height > 2 * kR && width > 2 * kR, GS_ERR_INVALID_ARGUMENT,
             "SSIM needs an image larger than its 11 x 11 window (got %d x %d)", height, width);
  GS_REQUIRE(image && target && ssim, GS_ERR_INVALID_ARGUMENT, "null pointer argument");
  const dim3 grid = fwd_grid(height, width);
  GS_REQUIRE(int64_t(grid.x) * grid.y <= kSsimPartials, GS_ERR_UNSUPPORTED,
             "image too large for the SSIM kernel (%d x %d)", height, width);
  GS_REQUIRE(workspace && workspace_bytes >= gs_ssim_workspace_bytes(height, width),
             GS_ERR_WORKSPACE, "workspace too small (%zu bytes, need %zu)", workspace_bytes,
             gs_ssim_workspace_bytes(height, width));
  float* gmap = static_cast<float*>(workspace);
  float* partial = reinterpret_cast<float*>(
      static_cast<char*>(workspace) + align_up(size_t(3) * height * width * 3 * sizeof(float)));
  const hipStream_t s = as_stream(stream);
  ssim_fwd_kernel<<<grid, kSsimThreads, 0, s>>>(image, target, height, width, window(), 1e-4f,
                                                9e-4f, gmap, partial);
  GS_TRY(check_launch("ssim_fwd"));
  const double count = 3.0 * double(height - 2 * kR) * double(width - 2 * kR);
  ssim_finish_kernel<<<1, kSsimThreads, 0, s>>>(partial, int(grid.x * grid.y), count, ssim);
  return check_launch("ssim_finish");
}

GS_API int gs_ssim_bwd(const float* image, const float* target, int32_t height, int32_t width,
                       const float* grad_ssim, const void* workspace, size_t workspace_bytes,
                       float* grad_image, void* stream) {
  clear_error();
  GS_REQUIRE(height > 2 * kR && width > 2 * kR, GS_ERR_INVALID_ARGUMENT,
             "SSIM needs an image larger than its 11 x 11 window (got %d x %d)", height, width);
  GS_REQUIRE(image && target && grad_ssim && grad_image, GS_ERR_INVALID_ARGUMENT,
             "null pointer argument");
  GS_REQUIRE(workspace && workspace_bytes >= gs_ssim_workspace_bytes(height, width),
             GS_ERR_WORKSPACE, "workspace too small (%zu bytes, need %zu)", workspace_bytes,
             gs_ssim_workspace_bytes(height, width));
  const float inv_count = float(1.0 / (3.0 * double(height - 2 * kR) * double(width - 2 * kR)));
  const dim3 grid(unsigned(ceil_div(width, kBW)), unsigned(ceil_div(height, kBH)));
  ssim_bwd_kernel<<<grid, kSsimThreads, 0, as_stream(stream)>>>(
      image, target, static_cast<const float*>(workspace), grad_ssim, inv_count, height, width,
      window(), grad_image);
  return check_launch("ssim_bwd");
}

}  // extern "C"
