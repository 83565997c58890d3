// One Adam step over up to kAdamMaxTensors parameter tensors in a single
// launch: the update torch.optim.Adam applies (its multi-tensor path, the
// default on GPUs) to the Gaussian parameters in the reference's training step
// (training/train.py:115, eps = 1e-15; step at train.py:151):
//   g  <- g + weight_decay * p                     (if weight_decay != 0)
//   m  <- lerp(m, g, 1 - beta1)
//   v  <- v * beta2 + (1 - beta2) * g * g
//   p  <- p + step_size * m / (sqrt(v) / bc2_sqrt + eps)
// with step_size = -lr / (1 - beta1^t) and bc2_sqrt = sqrt(1 - beta2^t)
// computed on the host in double precision per tensor, as torch does in
// Python.  Each element is read once (p, g, m, v) and written once (p, m, v):
// 28 bytes per parameter instead of the eight full passes of the op-by-op
// update.
#include <algorithm>
#include <cmath>

#include "common.h"

namespace gs {
namespace {

constexpr int kAdamMaxTensors = GS_ADAM_MAX_TENSORS;
constexpr int kAdamThreads = 256;
constexpr int kAdamVec = 4;                                 // floats per thread and chunk
constexpr int kAdamChunk = kAdamThreads * kAdamVec * 4;     // elements per workgroup

struct AdamTensorArg {
  float* p;
  const float* g;
  float* m;
  float* v;
  int64_t n;
  int64_t first_block;  // first workgroup of this tensor
  float step_size;      // -lr / (1 - beta1^t)
  float bc2_sqrt;       // sqrt(1 - beta2^t)
  int vec;              // all four pointers 16-byte aligned
};

struct AdamArgs {
  AdamTensorArg t[kAdamMaxTensors];
  int count;
  float one_minus_beta1, beta2, one_minus_beta2, eps, weight_decay;
};

__device__ __forceinline__ float lerp_small(float a, float b, float w) {
  // torch's lerp for weights below 0.5
  return a + w * (b - a);
}

__device__ __forceinline__ void adam_element(const AdamArgs& a, const AdamTensorArg& t, float& p,
                                             float g, float& m, float& v) {
  if (a.weight_decay != 0.0f) g = g + a.weight_decay * p;
  m = a.one_minus_beta1 < 0.5f ? lerp_small(m, g, a.one_minus_beta1)
                               : g - (g - m) * (1.0f - a.one_minus_beta1);
  v = v * a.beta2;
  v = v + a.one_minus_beta2 * (g * g);
  const float denom = sqrtf(v) / t.bc2_sqrt + a.eps;
  p = p + t.step_size * (m / denom);
}

__global__ __launch_bounds__(kAdamThreads) void adam_kernel(AdamArgs a) {
  int k = 0;
  while (k + 1 < a.count && int64_t(blockIdx.x) >= a.t[k + 1].first_block) ++k;
  const AdamTensorArg& t = a.t[k];
  const int64_t base = (int64_t(blockIdx.x) - t.first_block) * kAdamChunk;
  const int64_t end = min(base + int64_t(kAdamChunk), t.n);
  if (t.vec) {
    float4* p4 = reinterpret_cast<float4*>(t.p);
    const float4* g4 = reinterpret_cast<const float4*>(t.g);
    float4* m4 = reinterpret_cast<float4*>(t.m);
    float4* v4 = reinterpret_cast<float4*>(t.v);
    const int64_t vend = end & ~int64_t(3);
    for (int64_t i = base + int64_t(threadIdx.x) * 4; i < vend; i += kAdamThreads * 4) {
      const int64_t q = i >> 2;
      float4 p = p4[q], m = m4[q], v = v4[q];
      const float4 g = g4[q];
      adam_element(a, t, p.x, g.x, m.x, v.x);
      adam_element(a, t, p.y, g.y, m.y, v.y);
      adam_element(a, t, p.z, g.z, m.z, v.z);
      adam_element(a, t, p.w, g.w, m.w, v.w);
      p4[q] = p;
      m4[q] = m;
      v4[q] = v;
    }
    for (int64_t i = vend + threadIdx.x; i < end; i += kAdamThreads)
      adam_element(a, t, t.p[i], t.g[i], t.m[i], t.v[i]);
  } else {
    for (int64_t i = base + threadIdx.x; i < end; i += kAdamThreads)
      adam_element(a, t, t.p[i], t.g[i], t.m[i], t.v[i]);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" GS_API int gs_adam_step(const gs_adam_tensor* tensors, int32_t count, double beta1,
                                   double beta2, double eps, double weight_decay, void* stream) {
  clear_error();
  GS_REQUIRE(count >= 0 && count <= kAdamMaxTensors, GS_ERR_INVALID_ARGUMENT,
             "between 0 and %d tensors per step (got %d)", kAdamMaxTensors, count);
  GS_REQUIRE(count == 0 || tensors, GS_ERR_INVALID_ARGUMENT, "null tensor list");
  GS_REQUIRE(beta1 >= 0.0 && beta1 < 1.0 && beta2 >= 0.0 && beta2 < 1.0,
             GS_ERR_INVALID_ARGUMENT, "betas must lie in [0, 1)");
  AdamArgs a{};
  // Scalars reach the device as float, as torch's foreach ops convert them.
  a.one_minus_beta1 = float(1.0 - beta1);
  a.beta2 = float(beta2);
  a.one_minus_beta2 = float(1.0 - beta2);
  a.eps = float(eps);
  a.weight_decay = float(weight_decay);
  int64_t blocks = 0;
  int used = 0;
  for (int i = 0; i < count; ++i) {
    const gs_adam_tensor& s = tensors[i];
    GS_REQUIRE(s.numel >= 0, GS_ERR_INVALID_ARGUMENT, "tensor %d: negative size", i);
    if (s.numel == 0) continue;
    GS_REQUIRE(s.param && s.grad && s.exp_avg && s.exp_avg_sq, GS_ERR_INVALID_ARGUMENT,
               "tensor %d: null pointer", i);
    GS_REQUIRE(s.step >= 1, GS_ERR_INVALID_ARGUMENT, "tensor %d: step must be >= 1", i);
    AdamTensorArg& t = a.t[used++];
    t.p = s.param;
    t.g = s.grad;
    t.m = s.exp_avg;
    t.v = s.exp_avg_sq;
    t.n = s.numel;
    t.first_block = blocks;
    // Host arithmetic in double, as torch computes the scalars in Python.
    const double bc1 = 1.0 - std::pow(beta1, double(s.step));
    const double bc2 = 1.0 - std::pow(beta2, double(s.step));
    t.step_size = float((s.lr / bc1) * -1.0);
    t.bc2_sqrt = float(std::pow(bc2, 0.5));
    t.vec = aligned16(s.param) && aligned16(s.grad) && aligned16(s.exp_avg) &&
            aligned16(s.exp_avg_sq);
    blocks += ceil_div(s.numel, kAdamChunk);
  }
  a.count = used;
  if (used == 0) return GS_OK;
  GS_REQUIRE(blocks < (int64_t(1) << 31), GS_ERR_OVERFLOW, "too many parameters");
  adam_kernel<<<unsigned(blocks), kAdamThreads, 0, as_stream(stream)>>>(a);
  return check_launch("adam_step");
}
