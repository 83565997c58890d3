// Real spherical-harmonic basis up to degree 3 (band-major, m = -l..l) and its
// gradient with respect to the (unit) direction components.
//
// The basis is the normalised real SH of src/gaussian_splats/splats/utils.py:32-66,
// written in closed polynomial form (the constants are the standard
// normalisation factors sqrt((2l+1)/(4 pi) (l-|m|)!/(l+|m|)!) times sqrt(2) for
// m != 0, with the Condon-Shortley phase folded into the signs).  On the unit
// sphere the polynomials equal the recurrence; their tangential derivatives, which
// are all that survive the normalisation of the view direction, therefore agree too.
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace gs {
namespace sh {

constexpr float kC0 = 0.28209479177387814f;
constexpr float kC1 = 0.4886025119029199f;
constexpr float kC2a = 1.0925484305920792f;   // xy, yz, xz terms
constexpr float kC2b = 0.31539156525252005f;  // 2zz - xx - yy
constexpr float kC2c = 0.5462742152960396f;   // xx - yy
constexpr float kC3a = 0.5900435899266435f;   // y(3xx - yy), x(xx - 3yy)
constexpr float kC3b = 2.890611442640554f;    // xyz
constexpr float kC3c = 0.4570457994644658f;   // y(4zz - xx - yy), x(...)
constexpr float kC3d = 0.3731763325901154f;   // z(2zz - 3xx - 3yy)
constexpr float kC3e = 1.445305721320277f;    // z(xx - yy)

// basis[k] for k < K (K in {1, 4, 9, 16}).
template <int K>
__device__ __forceinline__ void basis(float x, float y, float z, float* b) {
  b[0] = kC0;
  if constexpr (K > 1) {
    b[1] = -kC1 * y;
    b[2] = kC1 * z;
    b[3] = -kC1 * x;
  }
  if constexpr (K > 4) {
    const float xx = x * x, yy = y * y, zz = z * z;
    b[4] = kC2a * (x * y);
    b[5] = -kC2a * (y * z);
    b[6] = kC2b * (2.0f * zz - xx - yy);
    b[7] = -kC2a * (x * z);
    b[8] = kC2c * (xx - yy);
    if constexpr (K > 9) {
      b[9] = -kC3a * y * (3.0f * xx - yy);
      b[10] = kC3b * (x * y) * z;
      b[11] = -kC3c * y * (4.0f * zz - xx - yy);
      b[12] = kC3d * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
      b[13] = -kC3c * x * (4.0f * zz - xx - yy);
      b[14] = kC3e * z * (xx - yy);
      b[15] = -kC3a * x * (xx - 3.0f * yy);
    }
  }
}

// Accumulates g . d(basis)/d(x, y, z) where g[k] = dL/d basis[k].
template <int K>
__device__ __forceinline__ void basis_vjp(float x, float y, float z, const float* g,
                                          float& gx, float& gy, float& gz) {
  gx = 0.0f;
  gy = 0.0f;
  gz = 0.0f;
  if constexpr (K > 1) {
    gy -= kC1 * g[1];
    gz += kC1 * g[2];
    gx -= kC1 * g[3];
  }
  if constexpr (K > 4) {
    const float xx = x * x, yy = y * y, zz = z * z;
    // b4 = C2a xy
    gx += kC2a * y * g[4];
    gy += kC2a * x * g[4];
    // b5 = -C2a yz
    gy -= kC2a * z * g[5];
    gz -= kC2a * y * g[5];
    // b6 = C2b (2zz - xx - yy)
    gx -= 2.0f * kC2b * x * g[6];
    gy -= 2.0f * kC2b * y * g[6];
    gz += 4.0f * kC2b * z * g[6];
    // b7 = -C2a xz
    gx -= kC2a * z * g[7];
    gz -= kC2a * x * g[7];
    // b8 = C2c (xx - yy)
    gx += 2.0f * kC2c * x * g[8];
    gy -= 2.0f * kC2c * y * g[8];
    if constexpr (K > 9) {
      // b9 = -C3a y (3xx - yy)
      gx -= kC3a * 6.0f * x * y * g[9];
      gy -= kC3a * 3.0f * (xx - yy) * g[9];
      // b10 = C3b xyz
      gx += kC3b * y * z * g[10];
      gy += kC3b * x * z * g[10];
      gz += kC3b * x * y * g[10];
      // b11 = -C3c y (4zz - xx - yy)
      gx += kC3c * 2.0f * x * y * g[11];
      gy -= kC3c * (4.0f * zz - xx - 3.0f * yy) * g[11];
      gz -= kC3c * 8.0f * y * z * g[11];
      // b12 = C3d z (2zz - 3xx - 3yy)
      gx -= kC3d * 6.0f * x * z * g[12];
      gy -= kC3d * 6.0f * y * z * g[12];
      gz += kC3d * (6.0f * zz - 3.0f * xx - 3.0f * yy) * g[12];
      // b13 = -C3c x (4zz - xx - yy)
      gx -= kC3c * (4.0f * zz - 3.0f * xx - yy) * g[13];
      gy += kC3c * 2.0f * x * y * g[13];
      gz -= kC3c * 8.0f * x * z * g[13];
      // b14 = C3e z (xx - yy)
      gx += kC3e * 2.0f * x * z * g[14];
      gy -= kC3e * 2.0f * y * z * g[14];
      gz += kC3e * (xx - yy) * g[14];
      // b15 = -C3a x (xx - 3yy)
      gx -= kC3a * 3.0f * (xx - yy) * g[15];
      gy += kC3a * 6.0f * x * y * g[15];
    }
  }
}

// One Gaussian's 3K coefficients ([K, 3] row-major) moved between global memory
// and registers, as dwordx4 accesses when 3K floats keep 16-byte alignment
// (K = 4 and 16; the caller checks the base pointer) and dword ones otherwise.
template <int K>
__device__ __forceinline__ void load_coefficients(const float* __restrict__ p, float* cf) {
  constexpr int F = 3 * K;
  if constexpr (F % 4 == 0) {
    const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int i = 0; i < F / 4; ++i) {
      const float4 v = q[i];
      cf[4 * i + 0] = v.x;
      cf[4 * i + 1] = v.y;
      cf[4 * i + 2] = v.z;
      cf[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < F; ++i) cf[i] = p[i];
  }
}

template <int K>
__device__ __forceinline__ void store_coefficients(float* __restrict__ p, const float* cf) {
  constexpr int F = 3 * K;
  if constexpr (F % 4 == 0) {
    float4* q = reinterpret_cast<float4*>(p);
#pragma unroll
    for (int i = 0; i < F / 4; ++i)
      q[i] = make_float4(cf[4 * i + 0], cf[4 * i + 1], cf[4 * i + 2], cf[4 * i + 3]);
  } else {
#pragma unroll
    for (int i = 0; i < F; ++i) p[i] = cf[i];
  }
}

// LDS layout of a staged coefficient block: row g holds Gaussian g's F
// floats.  When F is a multiple of 4 a row is C = F/4 16-byte chunks and the
// block moves between memory and LDS with 16-byte accesses on both sides:
//   - C odd: rows of C chunks, unpadded;
//   - C a multiple of 4: rows of C chunks, chunk j of row g in slot
//     j ^ chunk_swizzle(g) (the swizzle flips the two low bits, so it stays in
//     the row's aligned group of four slots);
//   - other even C: one chunk of padding (an odd row length).
// A wave reading chunk j of 8 (16) consecutive rows then touches 8 (16)
// distinct 16-byte bank groups of 32 (64) banks, and the stores of
// consecutive chunks of the block land in distinct groups too.  Otherwise
// (F % 4 != 0) rows of F + 1 floats (odd) for one-float accesses.
template <int F>
constexpr int row_stride() {
  return F % 4 != 0 ? F + 1 : ((F / 4) % 2 == 1 || (F / 4) % 4 == 0) ? F : F + 4;
}

template <int F>
__device__ __forceinline__ int chunk_swizzle(int g) {
  if constexpr (F % 4 == 0 && (F / 4) % 4 == 0) {
    return ((g >> 1) ^ (g >> 2)) & 3;
  } else {
    return 0;
  }
}

// Row g of a staged block, into registers.
template <int F>
__device__ __forceinline__ void row_load(const float* lds, int g, float* out) {
  const float* row = lds + g * row_stride<F>();
  if constexpr (F % 4 == 0) {
    const float4* r4 = reinterpret_cast<const float4*>(row);
    const int sw = chunk_swizzle<F>(g);
#pragma unroll
    for (int i = 0; i < F / 4; ++i) {
      const float4 v = r4[i ^ sw];
      out[4 * i + 0] = v.x;
      out[4 * i + 1] = v.y;
      out[4 * i + 2] = v.z;
      out[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < F; ++i) out[i] = row[i];
  }
}

// Registers into row g of a staged block.
template <int F>
__device__ __forceinline__ void row_store(float* lds, int g, const float* in) {
  float* row = lds + g * row_stride<F>();
  if constexpr (F % 4 == 0) {
    float4* r4 = reinterpret_cast<float4*>(row);
    const int sw = chunk_swizzle<F>(g);
#pragma unroll
    for (int i = 0; i < F / 4; ++i)
      r4[i ^ sw] = make_float4(in[4 * i + 0], in[4 * i + 1], in[4 * i + 2], in[4 * i + 3]);
  } else {
#pragma unroll
    for (int i = 0; i < F; ++i) row[i] = in[i];
  }
}

// Coefficient blocks staged through LDS: BLOCK Gaussians' F = 3K floats each
// (contiguous in memory, 16-byte aligned block start; LDS 16-byte aligned)
// move between memory and LDS rows (the layout above) with coalesced 16-byte
// loads.  For F % 4 == 0 each 16-byte chunk lands whole in one row (one
// 16-byte LDS store; lane i stores chunk i).  Otherwise a chunk can straddle two rows and is stored
// float by float.  In a full block every thread issues all of its loads
// before the first LDS store, so they are in flight together.  Called by all
// BLOCK threads; the caller synchronises around them.
template <int F, int BLOCK>
__device__ __forceinline__ void stage_block(const float* __restrict__ src, int nvalid, float* lds) {
  constexpr int S = row_stride<F>();
  const float4* src4 = reinterpret_cast<const float4*>(src);
  if constexpr (F % 4 == 0) {
    constexpr int C = F / 4;  // chunks per row; thread t's j-th chunk is t + j * BLOCK
    if (nvalid == BLOCK) {
      float4 v[C];
#pragma unroll
      for (int j = 0; j < C; ++j) v[j] = load_nt(src4 + threadIdx.x + j * BLOCK);
#pragma unroll
      for (int j = 0; j < C; ++j) {
        const int i = threadIdx.x + j * BLOCK;
        const int g = i / C;
        reinterpret_cast<float4*>(lds + g * S)[(i - g * C) ^ chunk_swizzle<F>(g)] = v[j];
      }
      return;
    }
    const int chunks = nvalid * C;
    for (int i = threadIdx.x; i < chunks; i += BLOCK) {
      const int g = i / C;
      reinterpret_cast<float4*>(lds + g * S)[(i - g * C) ^ chunk_swizzle<F>(g)] = load_nt(src4 + i);
    }
    return;
  }
  constexpr int kVec4 = BLOCK * F / 4;  // F * BLOCK is a multiple of 4 for BLOCK % 4 == 0
  constexpr int kPerThread = (kVec4 + BLOCK - 1) / BLOCK;
  if (nvalid == BLOCK) {
    float4 v[kPerThread];
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
      const int i = threadIdx.x + j * BLOCK;
      if (kVec4 % BLOCK == 0 || i < kVec4) v[j] = src4[i];
    }
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
      const int i = threadIdx.x + j * BLOCK;
      if (kVec4 % BLOCK == 0 || i < kVec4) {
        const float vals[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int e = i * 4 + t;
          const int g = e / F;
          lds[g * S + (e - g * F)] = vals[t];
        }
      }
    }
    return;
  }
  const int total = nvalid * F;
  for (int i = threadIdx.x; i * 4 < total; i += BLOCK) {
    const int f = i * 4;
    float vals[4];
    if (f + 4 <= total) {
      const float4 v = src4[i];
      vals[0] = v.x;
      vals[1] = v.y;
      vals[2] = v.z;
      vals[3] = v.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) vals[j] = (f + j < total) ? src[f + j] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = f + j;
      if (e < total) {
        const int g = e / F;
        lds[g * S + (e - g * F)] = vals[j];
      }
    }
  }
}

// The reverse of stage_block: LDS rows to memory with coalesced stores.
template <int F, int BLOCK>
__device__ __forceinline__ void unstage_block(float* __restrict__ dst, int nvalid, const float* lds) {
  constexpr int S = row_stride<F>();
  float4* dst4 = reinterpret_cast<float4*>(dst);
  if constexpr (F % 4 == 0) {
    constexpr int C = F / 4;
    const int chunks = nvalid * C;
    for (int i = threadIdx.x; i < chunks; i += BLOCK) {
      const int g = i / C;
      store_nt(reinterpret_cast<const float4*>(lds + g * S)[(i - g * C) ^ chunk_swizzle<F>(g)],
               dst4 + i);
    }
    return;
  }
  const int total = nvalid * F;
  for (int i = threadIdx.x; i * 4 < total; i += BLOCK) {
    float vals[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int e = i * 4 + t;
      const int g = e / F;
      vals[t] = e < total ? lds[g * S + (e - g * F)] : 0.0f;
    }
    if (i * 4 + 4 <= total) {
      dst4[i] = make_float4(vals[0], vals[1], vals[2], vals[3]);
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (i * 4 + t < total) dst[i * 4 + t] = vals[t];
    }
  }
}

}  // namespace sh
}  // namespace gs
