// Photometric L1 loss of the training step (training/train.py:137-138 of the
// reference): image' = clamp(image, 0, 1) when requested, loss =
// mean |image' - target|.
//
// Forward: one pass over image and target writes a per-workgroup partial sum
// and a one-byte code per element, code = sign(image' - target) where the
// clamp passes the gradient (0 <= image <= 1, or no clamp) and 0 elsewhere
// (sign(NaN) = 0, as torch.sign).  A single workgroup then adds the partial
// sums in a fixed order, so the loss is deterministic.
//
// Backward: grad_image = code * (grad_loss * (1 / numel)), the product the
// autograd chain mean -> abs -> sub -> clamp forms on the GPU (the mean's
// backward multiplies by the reciprocal of the element count), so the
// gradient is bit-identical to torch's.
#include <algorithm>

#include "common.h"

namespace gs {
namespace {

constexpr int kLossBlock = 256;
constexpr int kLossPartials = 1024;  // forward workgroups at most

__device__ __forceinline__ float loss_term(float x, float t, bool clamp, int& code) {
  bool pass = true;
  if (clamp) {
    pass = x >= 0.0f && x <= 1.0f;
    if (x == x) x = fminf(fmaxf(x, 0.0f), 1.0f);  // clamp keeps NaN
  }
  const float d = x - t;
  code = pass ? (d > 0.0f) - (d < 0.0f) : 0;
  return fabsf(d);
}

__device__ __forceinline__ float block_sum(float v, float* scratch) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wid] = v;
  __syncthreads();
  float s = 0.0f;
  if (threadIdx.x == 0)
    for (int w = 0; w < kLossBlock / 64; ++w) s += scratch[w];
  return s;
}

// `vec`: image, target and code allow 16- and 4-byte vector accesses.
__global__ __launch_bounds__(kLossBlock) void l1_fwd_kernel(const float* __restrict__ image,
                                                            const float* __restrict__ target,
                                                            int64_t numel, bool clamp, bool vec,
                                                            int8_t* __restrict__ code,
                                                            float* __restrict__ partial) {
  __shared__ float scratch[kLossBlock / 64];
  float acc = 0.0f;
  const int64_t stride = int64_t(gridDim.x) * kLossBlock;
  const int64_t t0 = int64_t(blockIdx.x) * kLossBlock + threadIdx.x;
  int64_t tail = 0;
  if (vec) {
    const int64_t n4 = numel / 4;
    const float4* im4 = reinterpret_cast<const float4*>(image);
    const float4* tg4 = reinterpret_cast<const float4*>(target);
    char4* c4 = reinterpret_cast<char4*>(code);
    for (int64_t i = t0; i < n4; i += stride) {
      const float4 x = load_nt(im4 + i), t = load_nt(tg4 + i);  // read once
      int c0, c1, c2, c3;
      acc += loss_term(x.x, t.x, clamp, c0);
      acc += loss_term(x.y, t.y, clamp, c1);
      acc += loss_term(x.z, t.z, clamp, c2);
      acc += loss_term(x.w, t.w, clamp, c3);
      c4[i] = make_char4(char(c0), char(c1), char(c2), char(c3));
    }
    tail = n4 * 4;
  }
  for (int64_t i = tail + t0; i < numel; i += stride) {
    int c;
    acc += loss_term(image[i], target[i], clamp, c);
    code[i] = int8_t(c);
  }
  const float s = block_sum(acc, scratch);
  if (threadIdx.x == 0) partial[blockIdx.x] = s;
}

__global__ __launch_bounds__(kLossBlock) void l1_finish_kernel(const float* __restrict__ partial,
                                                               int blocks, int64_t numel,
                                                               float* __restrict__ loss) {
  __shared__ double scratch[kLossBlock / 64];
  double acc = 0.0;
  for (int i = threadIdx.x; i < blocks; i += kLossBlock) acc += double(partial[i]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int w = 0; w < kLossBlock / 64; ++w) s += scratch[w];
    loss[0] = float(s / double(numel));
  }
}

__global__ __launch_bounds__(kLossBlock) void l1_bwd_kernel(const int8_t* __restrict__ code,
                                                            const float* __restrict__ grad_loss,
                                                            float inv_numel, int64_t numel,
                                                            bool vec, float* __restrict__ grad) {
  const float s = grad_loss[0] * inv_numel;
  const int64_t stride = int64_t(gridDim.x) * kLossBlock;
  const int64_t t0 = int64_t(blockIdx.x) * kLossBlock + threadIdx.x;
  int64_t tail = 0;
  if (vec) {
    const int64_t n4 = numel / 4;
    const char4* c4 = reinterpret_cast<const char4*>(code);
    float4* g4 = reinterpret_cast<float4*>(grad);
    for (int64_t i = t0; i < n4; i += stride) {
      const char4 c = c4[i];
      g4[i] = make_float4(float(c.x) * s, float(c.y) * s, float(c.z) * s, float(c.w) * s);
    }
    tail = n4 * 4;
  }
  for (int64_t i = tail + t0; i < numel; i += stride) grad[i] = float(code[i]) * s;
}

// Regularisers of the training step (train.py:140-141): the means of
// sigmoid(opacity) over N and of exp(scale) over 3N, two partial sums per
// workgroup, added in a fixed order by reg_finish_kernel.
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

__global__ __launch_bounds__(kLossBlock) void reg_fwd_kernel(const float* __restrict__ opacity,
                                                             const float* __restrict__ scale,
                                                             int64_t n, float* __restrict__ partial) {
  __shared__ float scratch[kLossBlock / 64];
  const int64_t stride = int64_t(gridDim.x) * kLossBlock;
  const int64_t t0 = int64_t(blockIdx.x) * kLossBlock + threadIdx.x;
  float so = 0.0f, ss = 0.0f;
  for (int64_t i = t0; i < n; i += stride) so += sigmoid(opacity[i]);
  for (int64_t i = t0; i < 3 * n; i += stride) ss += expf(scale[i]);
  const float bo = block_sum(so, scratch);
  __syncthreads();
  const float bs = block_sum(ss, scratch);
  if (threadIdx.x == 0) {
    partial[2 * blockIdx.x] = bo;
    partial[2 * blockIdx.x + 1] = bs;
  }
}

__global__ __launch_bounds__(kLossBlock) void reg_finish_kernel(const float* __restrict__ partial,
                                                                int blocks, int64_t n,
                                                                float* __restrict__ out) {
  __shared__ double scratch[2][kLossBlock / 64];
  double ao = 0.0, as = 0.0;
  for (int i = threadIdx.x; i < blocks; i += kLossBlock) {
    ao += double(partial[2 * i]);
    as += double(partial[2 * i + 1]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    ao += __shfl_xor(ao, o, 64);
    as += __shfl_xor(as, o, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    scratch[0][threadIdx.x >> 6] = ao;
    scratch[1][threadIdx.x >> 6] = as;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double so = 0.0, ss = 0.0;
    for (int w = 0; w < kLossBlock / 64; ++w) {
      so += scratch[0][w];
      ss += scratch[1][w];
    }
    out[0] = float(so / double(n));
    out[1] = float(ss / (3.0 * double(n)));
  }
}

// Autograd's gradients of the two means: (g0 (1/N)) (1 - y) y with
// y = sigmoid(opacity), and (g1 (1/3N)) exp(scale).
__global__ __launch_bounds__(kLossBlock) void reg_bwd_kernel(
    const float* __restrict__ opacity, const float* __restrict__ scale, int64_t n,
    const float* __restrict__ grad_out, float inv_n, float inv_3n,
    float* __restrict__ grad_opacity, float* __restrict__ grad_scale) {
  const float go = grad_out[0] * inv_n, gs_ = grad_out[1] * inv_3n;
  const int64_t stride = int64_t(gridDim.x) * kLossBlock;
  const int64_t t0 = int64_t(blockIdx.x) * kLossBlock + threadIdx.x;
  for (int64_t i = t0; i < n; i += stride) {
    const float y = sigmoid(opacity[i]);
    grad_opacity[i] = go * (1.0f - y) * y;
  }
  for (int64_t i = t0; i < 3 * n; i += stride) grad_scale[i] = gs_ * expf(scale[i]);
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int loss_blocks(int64_t numel) {
  return int(std::max<int64_t>(1, std::min<int64_t>(kLossPartials, ceil_div(numel, 4 * kLossBlock * 4))));
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" {

GS_API size_t gs_l1_loss_workspace_bytes(int64_t numel) {
  (void)numel;
  return size_t(kLossPartials) * sizeof(float);
}

GS_API int gs_l1_loss_fwd(const float* image, const float* target, int64_t numel, int32_t clamp,
                          float* loss, int8_t* code, void* workspace, size_t workspace_bytes,
                          void* stream) {
  clear_error();
  GS_REQUIRE(numel >= 0, GS_ERR_INVALID_ARGUMENT, "numel must be non-negative");
  GS_REQUIRE(loss && (numel == 0 || (image && target && code)), GS_ERR_INVALID_ARGUMENT,
             "null pointer argument");
  GS_REQUIRE(workspace && workspace_bytes >= gs_l1_loss_workspace_bytes(numel),
             GS_ERR_WORKSPACE, "workspace too small (%zu bytes, need %zu)", workspace_bytes,
             gs_l1_loss_workspace_bytes(numel));
  const hipStream_t s = as_stream(stream);
  float* partial = static_cast<float*>(workspace);
  const int blocks = loss_blocks(numel);
  const bool vec = aligned(image, 16) && aligned(target, 16) && aligned(code, 4);
  l1_fwd_kernel<<<blocks, kLossBlock, 0, s>>>(image, target, numel, clamp != 0, vec, code,
                                              partial);
  GS_TRY(check_launch("l1_loss_fwd"));
  // An empty input gives 0 / 0 = NaN, as torch's mean of an empty tensor.
  l1_finish_kernel<<<1, kLossBlock, 0, s>>>(partial, blocks, numel, loss);
  return check_launch("l1_loss_finish");
}

GS_API int gs_l1_loss_bwd(const int8_t* code, const float* grad_loss, int64_t numel,
                          float* grad_image, void* stream) {
  clear_error();
  GS_REQUIRE(numel >= 0, GS_ERR_INVALID_ARGUMENT, "numel must be non-negative");
  if (numel == 0) return GS_OK;
  GS_REQUIRE(code && grad_loss && grad_image, GS_ERR_INVALID_ARGUMENT, "null pointer argument");
  const bool vec = aligned(code, 4) && aligned(grad_image, 16);
  const float inv_numel = 1.0f / float(numel);
  l1_bwd_kernel<<<loss_blocks(numel), kLossBlock, 0, as_stream(stream)>>>(code, grad_loss,
                                                                          inv_numel, numel, vec,
                                                                          grad_image);
  return check_launch("l1_loss_bwd");
}

GS_API size_t gs_splat_regularizers_workspace_bytes(int64_t n) {
  (void)n;
  return size_t(2 * kLossPartials) * sizeof(float);
}

GS_API int gs_splat_regularizers_fwd(const float* opacity, const float* scale, int64_t n,
                                     float* out, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0, GS_ERR_INVALID_ARGUMENT, "n must be non-negative");
  GS_REQUIRE(out && (n == 0 || (opacity && scale)), GS_ERR_INVALID_ARGUMENT,
             "null pointer argument");
  GS_REQUIRE(workspace && workspace_bytes >= gs_splat_regularizers_workspace_bytes(n),
             GS_ERR_WORKSPACE, "workspace too small (%zu bytes, need %zu)", workspace_bytes,
             gs_splat_regularizers_workspace_bytes(n));
  const hipStream_t s = as_stream(stream);
  float* partial = static_cast<float*>(workspace);
  const int blocks = loss_blocks(3 * n);
  reg_fwd_kernel<<<blocks, kLossBlock, 0, s>>>(opacity, scale, n, partial);
  GS_TRY(check_launch("regularizers_fwd"));
  // n = 0 gives 0 / 0 = NaN for both means, as torch's mean of an empty tensor.
  reg_finish_kernel<<<1, kLossBlock, 0, s>>>(partial, blocks, n, out);
  return check_launch("regularizers_finish");
}

GS_API int gs_splat_regularizers_bwd(const float* opacity, const float* scale, int64_t n,
                                     const float* grad_out, float* grad_opacity,
                                     float* grad_scale, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0, GS_ERR_INVALID_ARGUMENT, "n must be non-negative");
  if (n == 0) return GS_OK;
  GS_REQUIRE(opacity && scale && grad_out && grad_opacity && grad_scale, GS_ERR_INVALID_ARGUMENT,
             "null pointer argument");
  const float inv_n = 1.0f / float(n), inv_3n = 1.0f / float(3 * n);
  reg_bwd_kernel<<<loss_blocks(3 * n), kLossBlock, 0, as_stream(stream)>>>(
      opacity, scale, n, grad_out, inv_n, inv_3n, grad_opacity, grad_scale);
  return check_launch("regularizers_bwd");
}

}  // extern "C"
