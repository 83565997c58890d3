// Gaussian-splat PLY records <-> parameter tensors on the GPU.
//
// The reference stores a scene as one binary PLY "vertex" element whose
// float32 properties are, per Gaussian, x y z nx ny nz f_dc_0..2
// f_rest_0..3(K-1)-1 opacity scale_0..2 rot_0..3, with the higher-order SH
// coefficients channel-major: f_rest_{c (K-1) + k - 1} = color[k][c]
// (src/gaussian_splats/splats/ply.py:12-52 writes it, ply.py:55-89 reads it
// by property name, so files of other tools with other property orders,
// extra properties and no normals load too).
//
// Loading uploads the file's vertex block unchanged and splits it here:
// each workgroup stages the bytes of G consecutive records in LDS with
// coalesced 16-byte loads, then writes every output tensor's slice of those
// G Gaussians with consecutive lanes on consecutive floats.  A host-built
// table gives, for each output float of a Gaussian (canonical order: mean 3,
// normals 3, rotation 4, scale 3, opacity 1, color 3K coefficient-major), the
// byte offset of its property in the record, or -1 for a zero.  Records may
// have any size (properties of other types are skipped by their offsets) and
// either byte order.  Saving is the inverse: inputs are staged in LDS per
// workgroup and the records are written with coalesced dword stores.
#include <algorithm>

#include "common.h"

namespace gs {
namespace {

constexpr int kPlyBlock = 256;
constexpr int kPlyStageBytes = 32768;  // LDS staging per workgroup

struct UnpackArgs {
  const uint8_t* records;
  int64_t n;
  int64_t total_bytes;  // n * record_bytes
  int record_bytes;
  int group;            // Gaussians per workgroup
  int big_endian;
  int fields;           // 14 + 3K
  int offset[GS_PLY_MAX_FIELDS];
  float* out[6];
  int width[6];
  int first[6];  // first field of each output tensor
};

__device__ __forceinline__ uint32_t bswap32(uint32_t v) {
  return (v >> 24) | ((v >> 8) & 0xff00u) | ((v << 8) & 0xff0000u) | (v << 24);
}

__global__ __launch_bounds__(kPlyBlock) void ply_unpack_kernel(UnpackArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t stage[];
  const int64_t g0 = int64_t(blockIdx.x) * a.group;
  const int64_t gcount = min(int64_t(a.group), a.n - g0);
  const int64_t lo = g0 * a.record_bytes;
  const int64_t hi = lo + gcount * a.record_bytes;
  const int64_t lo16 = lo & ~int64_t(15);
  const int64_t total16 = a.total_bytes & ~int64_t(15);
  // Bulk: whole 16-byte words inside the buffer (the buffer starts 16-byte
  // aligned, checked on the host).
  const int64_t bulk_end = min((hi + 15) & ~int64_t(15), total16);
  const uint4* src4 = reinterpret_cast<const uint4*>(a.records + lo16);
  uint4* dst4 = reinterpret_cast<uint4*>(stage);
  const int words = bulk_end > lo16 ? int((bulk_end - lo16) >> 4) : 0;
  for (int i = threadIdx.x; i < words; i += kPlyBlock) dst4[i] = src4[i];
  // Tail: the bytes after the last whole word of the buffer (last group only).
  for (int64_t b = max(lo16, total16) + threadIdx.x; b < hi; b += kPlyBlock)
    stage[b - lo16] = a.records[b];
  __syncthreads();

  const int64_t rel0 = lo - lo16;
  const bool word_aligned = ((a.record_bytes | int(rel0)) & 3) == 0;
  for (int t = 0; t < 6; ++t) {
    float* out = a.out[t];
    const int w = a.width[t];
    const int count = int(gcount) * w;
    for (int e = threadIdx.x; e < count; e += kPlyBlock) {
      const int g = e / w;
      const int off = a.offset[a.first[t] + (e - g * w)];
      uint32_t bits = 0;
      if (off >= 0) {
        const int64_t p = rel0 + int64_t(g) * a.record_bytes + off;
        if (word_aligned && (off & 3) == 0) {
          bits = *reinterpret_cast<const uint32_t*>(stage + p);
        } else {
          bits = uint32_t(stage[p]) | (uint32_t(stage[p + 1]) << 8) |
                 (uint32_t(stage[p + 2]) << 16) | (uint32_t(stage[p + 3]) << 24);
        }
        if (a.big_endian) bits = bswap32(bits);
      }
      out[g0 * w + e] = __uint_as_float(bits);
    }
  }
}

struct PackArgs {
  const float* in[6];  // in[1] (normals) may be null: zeros
  int width[6];
  int64_t n;
  int record_floats;  // 14 + 3K
  int group;
  int k;
  float* records;
};

// Record position of canonical field j (the reference's property order).
__device__ __forceinline__ int record_slot(int t, int j, int k) {
  switch (t) {
    case 0: return j;           // x y z
    case 1: return 3 + j;       // nx ny nz
    case 2: return 10 + 3 * k + j;  // rot_0..3 after opacity and scales
    case 3: return 7 + 3 * k + j;   // scale_0..2
    case 4: return 6 + 3 * k;       // opacity
    default: {                      // color[kk][c]
      const int kk = j / 3, c = j - kk * 3;
      return kk == 0 ? 6 + c : 9 + c * (k - 1) + (kk - 1);
    }
  }
}

__global__ __launch_bounds__(kPlyBlock) void ply_pack_kernel(PackArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t stage_bytes[];
  float* stage = reinterpret_cast<float*>(stage_bytes);
  const int64_t g0 = int64_t(blockIdx.x) * a.group;
  const int gcount = int(min(int64_t(a.group), a.n - g0));
  const int rf = a.record_floats;
  for (int t = 0; t < 6; ++t) {
    const float* in = a.in[t];
    const int w = a.width[t];
    const int count = gcount * w;
    for (int e = threadIdx.x; e < count; e += kPlyBlock) {
      const int g = e / w;
      const int j = e - g * w;
      stage[g * rf + record_slot(t, j, a.k)] = in ? in[g0 * w + e] : 0.0f;
    }
  }
  __syncthreads();
  float* dst = a.records + g0 * rf;
  const int count = gcount * rf;
  for (int e = threadIdx.x; e < count; e += kPlyBlock) dst[e] = stage[e];
}

int ply_group(int record_bytes) {
  return std::max(1, std::min(kPlyBlock, (kPlyStageBytes - 32) / std::max(record_bytes, 1)));
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" {

GS_API int gs_ply_unpack(const void* records, int64_t n, int32_t record_bytes,
                         const int32_t* field_offsets, int32_t big_endian, int32_t sh_coeffs,
                         float* mean, float* normals, float* rotation, float* scale,
                         float* opacity, float* color, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0, GS_ERR_INVALID_ARGUMENT, "n must be non-negative");
  GS_REQUIRE(sh_coeffs >= 1 && 14 + 3 * sh_coeffs <= GS_PLY_MAX_FIELDS, GS_ERR_UNSUPPORTED,
             "sh_coeffs must be in [1, %d] (got %d)", (GS_PLY_MAX_FIELDS - 14) / 3, sh_coeffs);
  GS_REQUIRE(record_bytes >= 4 && record_bytes <= kPlyStageBytes - 32, GS_ERR_UNSUPPORTED,
             "record_bytes must be in [4, %d] (got %d)", kPlyStageBytes - 32, record_bytes);
  GS_REQUIRE(field_offsets, GS_ERR_INVALID_ARGUMENT, "null field_offsets");
  if (n == 0) return GS_OK;
  GS_REQUIRE(records && mean && normals && rotation && scale && opacity && color,
             GS_ERR_INVALID_ARGUMENT, "null pointer argument");
  GS_REQUIRE((reinterpret_cast<uintptr_t>(records) & 15) == 0, GS_ERR_INVALID_ARGUMENT,
             "records must be 16-byte aligned");
  GS_REQUIRE(n <= INT64_MAX / record_bytes, GS_ERR_OVERFLOW, "n * record_bytes overflows");
  UnpackArgs a{};
  a.records = static_cast<const uint8_t*>(records);
  a.n = n;
  a.total_bytes = n * record_bytes;
  a.record_bytes = record_bytes;
  a.group = ply_group(record_bytes);
  a.big_endian = big_endian != 0;
  a.fields = 14 + 3 * sh_coeffs;
  for (int f = 0; f < a.fields; ++f) {
    const int off = field_offsets[f];
    GS_REQUIRE(off >= -1 && off <= record_bytes - 4, GS_ERR_INVALID_ARGUMENT,
               "field %d: offset %d outside a %d-byte record", f, off, record_bytes);
    a.offset[f] = off;
  }
  float* outs[6] = {mean, normals, rotation, scale, opacity, color};
  const int widths[6] = {3, 3, 4, 3, 1, 3 * sh_coeffs};
  int first = 0;
  for (int t = 0; t < 6; ++t) {
    a.out[t] = outs[t];
    a.width[t] = widths[t];
    a.first[t] = first;
    first += widths[t];
  }
  const int64_t blocks = ceil_div(n, a.group);
  GS_REQUIRE(blocks <= INT32_MAX, GS_ERR_OVERFLOW, "too many Gaussians");
  const size_t lds = align_up(size_t(a.group) * record_bytes + 32, 16);
  launch_timed(ply_unpack_kernel, int(blocks), kPlyBlock, uint32_t(lds), as_stream(stream), a);
  return check_launch("ply_unpack");
}

GS_API int gs_ply_pack(const float* mean, const float* normals, const float* rotation,
                       const float* scale, const float* opacity, const float* color, int64_t n,
                       int32_t sh_coeffs, void* records, void* stream) {
  clear_error();
  GS_REQUIRE(n >= 0, GS_ERR_INVALID_ARGUMENT, "n must be non-negative");
  GS_REQUIRE(sh_coeffs >= 1 && 14 + 3 * sh_coeffs <= GS_PLY_MAX_FIELDS, GS_ERR_UNSUPPORTED,
             "sh_coeffs must be in [1, %d] (got %d)", (GS_PLY_MAX_FIELDS - 14) / 3, sh_coeffs);
  if (n == 0) return GS_OK;
  GS_REQUIRE(records && mean && rotation && scale && opacity && color, GS_ERR_INVALID_ARGUMENT,
             "null pointer argument");
  PackArgs a{};
  const float* ins[6] = {mean, normals, rotation, scale, opacity, color};
  const int widths[6] = {3, 3, 4, 3, 1, 3 * sh_coeffs};
  for (int t = 0; t < 6; ++t) {
    a.in[t] = ins[t];
    a.width[t] = widths[t];
  }
  a.n = n;
  a.k = sh_coeffs;
  a.record_floats = 14 + 3 * sh_coeffs;
  a.group = ply_group(4 * a.record_floats);
  a.records = static_cast<float*>(records);
  const int64_t blocks = ceil_div(n, a.group);
  GS_REQUIRE(blocks <= INT32_MAX, GS_ERR_OVERFLOW, "too many Gaussians");
  const size_t lds = size_t(a.group) * a.record_floats * sizeof(float);
  launch_timed(ply_pack_kernel, int(blocks), kPlyBlock, uint32_t(lds), as_stream(stream), a);
  return check_launch("ply_pack");
}

}  // extern "C"
