// Single-pass building blocks: a stable LSD radix sort whose passes each read
// and write the data once (digit offsets by decoupled look-back), and a
// single-kernel exclusive scan with the same look-back.
//
// Look-back protocol.  Workgroups take a ticket from an atomic counter, so a
// workgroup's predecessors already run or have finished.  Each publishes, per
// digit (or once, for the scan), a 64-bit status word: bits 63..62 are the flag
// (0 not ready, 1 aggregate = its own count, 2 prefix = inclusive sum over
// workgroups 0..b) and bits 61..0 the value.  A workgroup publishes its
// aggregate first, then walks back summing aggregates until it meets a prefix,
// then publishes its own prefix.  Every wait ends because predecessors never
// wait on successors; a spin limit turns a broken invariant into an error flag
// instead of a hang.
#pragma once

#include "block_scan.h"
#include "common.h"

namespace gs {
namespace sweep {

constexpr int kBlock = 256;
constexpr int kItems = 16;  // per thread: 4096 keys per tile keeps the look-back chain short
constexpr int kTile = kBlock * kItems;  // elements per workgroup
constexpr int kMaxPasses = 8;
constexpr int kMaxDigitBits = 8;  // digits of up to 8 bits (256 buckets)
constexpr int kHistStride = 1 << kMaxDigitBits;  // histogram words per pass
constexpr uint64_t kFlagAggregate = 1ull << 62;
constexpr uint64_t kFlagPrefix = 2ull << 62;
constexpr uint64_t kValueMask = (1ull << 62) - 1;
constexpr int kSpinLimit = 1 << 20;

struct Plan {
  int passes;
  int shift[kMaxPasses];
  int bits[kMaxPasses];
  // With `remap`, the histogram and the first pass sort key' = min(key -
  // base, cap) (keys below `base` wrap to large values and clamp to `cap`),
  // and the first pass writes key' for the later ones.
  bool remap;
  uint64_t base;
  uint64_t cap;
};

// Splits [0, end_bit) into ceil(end_bit / max_bits) passes of near-equal
// width (max_bits <= kMaxDigitBits).
inline Plan make_plan(int end_bit, int max_bits = 8) {
  Plan p{};
  const int total = end_bit <= 0 ? 1 : end_bit;
  p.passes = (total + max_bits - 1) / max_bits;
  int shift = 0;
  for (int i = 0; i < p.passes; ++i) {
    const int left = p.passes - i;
    const int bits = (total - shift + left - 1) / left;
    p.shift[i] = shift;
    p.bits[i] = bits;
    shift += bits;
  }
  return p;
}

__device__ __forceinline__ void store_status(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t load_status(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sum of the values of workgroups [0, b) in column `col` of a [*, stride]
// status array, walking back until an inclusive prefix is found.  The
// statuses of kLookBackBatch predecessors are requested together, so a walk
// over workgroups that have published only their aggregates takes one
// memory round trip per kLookBackBatch of them; they are consumed in order,
// and the walk resumes at the first one not yet published.
constexpr int kLookBackBatch = 4;
__device__ inline uint64_t look_back(const uint64_t* status, int64_t stride, int b, int col,
                                     uint32_t* err) {
  uint64_t excl = 0;
  int spins = 0;
  for (int k = b - 1; k >= 0;) {
    uint64_t v[kLookBackBatch];
#pragma unroll
    for (int i = 0; i < kLookBackBatch; ++i)  // before workgroup 0: prefix 0
      v[i] = k - i >= 0 ? load_status(status + int64_t(k - i) * stride + col) : kFlagPrefix;
    int used = 0;
#pragma unroll
    for (int i = 0; i < kLookBackBatch; ++i) {
      const uint64_t flag = v[i] >> 62;
      if (flag == 0) break;
      excl += v[i] & kValueMask;
      if (flag == 2) return excl;
      ++used;
    }
    if (used < kLookBackBatch) {  // predecessor k - used has not published yet
      if (++spins > kSpinLimit) {
        atomicOr(err, kDeviceFlagSpinLimit);
        return excl;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    k -= used;
  }
  return excl;
}

// The same walk for a single column (stride 1) by a whole wave: lane i reads
// the status of workgroup k0 - i, so one memory round trip covers 64
// predecessors.  Wave-uniform result.
__device__ inline uint64_t wave_look_back(const uint64_t* status, int b, uint32_t* err) {
  const int lane = __lane_id();
  uint64_t excl = 0;
  int spins = 0;
  for (int k0 = b - 1; k0 >= 0;) {
    const int k = k0 - lane;
    const uint64_t v = k >= 0 ? load_status(status + k) : kFlagPrefix;  // before 0: prefix 0
    const uint64_t prefix = __ballot((v >> 62) == 2);
    const uint64_t waiting = __ballot((v >> 62) == 0);
    const int first = prefix ? __builtin_ctzll(prefix) : 63;  // lanes 0..first are needed
    const uint64_t needed = first == 63 ? ~0ull : ((1ull << (first + 1)) - 1);
    if (waiting & needed) {
      if (++spins > kSpinLimit) {
        if (lane == 0) atomicOr(err, kDeviceFlagSpinLimit);
        return excl;
      }
      __builtin_amdgcn_s_sleep(2);
      continue;
    }
    uint64_t part = lane <= first ? (v & kValueMask) : 0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o, 64);
    excl += part;
    if (prefix) return excl;
    k0 -= 64;
  }
  return excl;
}

// Zeroes `words` 64-bit words and `small` 32-bit words (tickets, histograms).
__global__ __launch_bounds__(kBlock) inline void clear_kernel(uint64_t* big, int64_t words,
                                                              uint32_t* small, int small_words) {
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < words; i += stride) big[i] = 0;
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < small_words; i += kBlock) small[i] = 0;
}

// Digit histograms of every pass in one read of the keys.  The lanes of a
// wave that share a digit are found with eight ballots and counted by one LDS
// atomic from the lowest of them: keys that agree in a digit (the exponent
// byte of depths in one octave, the all-ones key of culled Gaussians) would
// otherwise serialise 64 same-address atomics per wave.  SPREAD (depth keys:
// the bits of positive floats, ~0 for culled Gaussians): only the last pass,
// the exponent byte, takes the ballots; the lower passes' digits are mantissa
// bytes, spread over the bins, and each lane adds its own with one LDS
// atomic, except the all-ones keys, counted once per wave.
constexpr int kHistBlock = 1024;
constexpr int kHistKeys = 4;
template <typename K, bool SPREAD = false>
__global__ __launch_bounds__(kHistBlock) void hist_kernel(const K* __restrict__ keys, int64_t n,
                                                      Plan plan, uint32_t* __restrict__ hist) {
  __shared__ uint32_t h[kMaxPasses * kHistStride];
  for (int i = threadIdx.x; i < plan.passes * kHistStride; i += kHistBlock) h[i] = 0;
  __syncthreads();
  const int lane = __lane_id();
  const int64_t stride = int64_t(gridDim.x) * kHistBlock;
  // Each round requests a thread's next kHistKeys keys together, then counts
  // them (one dependent round trip per round, not per key).
  for (int64_t i0 = int64_t(blockIdx.x) * kHistBlock + threadIdx.x; i0 - threadIdx.x < n;
       i0 += stride * kHistKeys) {
    K k[kHistKeys];
#pragma unroll
    for (int u = 0; u < kHistKeys; ++u) {
      const int64_t i = i0 + u * stride;
      k[u] = i < n ? keys[i] : K(0);
      if (plan.remap) k[u] = min(K(k[u] - K(plan.base)), K(plan.cap));
    }
#pragma unroll
    for (int u = 0; u < kHistKeys; ++u) {
      const bool ok = i0 + u * stride < n;
      const uint64_t active = __ballot(ok);
      if (!active) continue;
      // The pass loops run over the constant kKeyPasses (a key of B bytes
      // has at most B passes of at most eight bits) with wave-uniform guards:
      // constant indices keep the plan's shifts and masks in registers (a
      // runtime index into the kernel argument reloaded them with a dependent
      // scalar load per key and pass).
      constexpr int kKeyPasses = int(sizeof(K)) < kMaxPasses ? int(sizeof(K)) : kMaxPasses;
      int first_ballot_pass = 0;
      if constexpr (SPREAD) {
        const bool ones = k[u] == (plan.remap ? K(plan.cap) : ~K(0));
        const uint32_t n_ones = uint32_t(__popcll(__ballot(ok && ones)));
#pragma unroll
        for (int p = 0; p + 1 < kKeyPasses; ++p) {
          if (p + 1 >= plan.passes) break;
          const uint32_t d = uint32_t(k[u] >> plan.shift[p]) & ((1u << plan.bits[p]) - 1u);
          if (ok && !ones) atomicAdd(&h[p * kHistStride + d], 1u);
          if (lane == 0 && n_ones)
            atomicAdd(&h[p * kHistStride + (1u << plan.bits[p]) - 1u], n_ones);
        }
        first_ballot_pass = plan.passes - 1;
      }
#pragma unroll
      for (int p = 0; p < kKeyPasses; ++p) {
        if (p >= plan.passes) break;
        if (p < first_ballot_pass) continue;
        const uint32_t d = uint32_t(k[u] >> plan.shift[p]) & ((1u << plan.bits[p]) - 1u);
        // Active lanes with the same digit (digits have at most eight bits).
        uint64_t peers = active;
#pragma unroll
        for (int bit = 0; bit < kMaxDigitBits; ++bit) {
          const bool set = (d >> bit) & 1u;
          const uint64_t ones = __ballot(set);
          peers &= set ? ones : ~ones;
        }
        if (ok && lane == __builtin_ctzll(peers))
          atomicAdd(&h[p * kHistStride + d], uint32_t(__popcll(peers)));
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < plan.passes * kHistStride; i += kHistBlock)
    if (h[i]) atomicAdd(&hist[i], h[i]);
}

// Stable rank of each of a wave's 64 items among the items of the same digit:
// `peers` = lanes whose digit matches (one ballot per digit bit; a lane keeps
// the ballot where its own bit is set and its complement where it is clear),
// rank in the wave = peers below this lane (mbcnt), and the running count of
// the digit in this wave's segment lives in LDS.  All peers write the same new
// count, so no leader election is needed; a wave's LDS accesses execute in
// program order, so item i+1 sees item i's counts.
template <int BITS, bool FULL, int ITEMS = kItems>
__device__ __forceinline__ void rank_items(const uint32_t* digits, int n_valid_from_seg,
                                           uint32_t* wcnt, uint32_t* rank) {
  const int lane = __lane_id();
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const uint32_t d = digits[i];
    bool valid = true;
    uint32_t plo = ~0u, phi = ~0u;
    if (!FULL) {
      valid = i * 64 + lane < n_valid_from_seg;
      const uint64_t vm = __ballot(valid);
      plo = uint32_t(vm);
      phi = uint32_t(vm >> 32);
    }
    uint32_t m[BITS];
    uint64_t ones[BITS];
#pragma unroll
    for (int bit = 0; bit < BITS; ++bit) {
      m[bit] = uint32_t(int32_t(d << (31 - bit)) >> 31);  // v_bfe_i32: 0 or all ones
      // Opaque, so that the ballot compares m itself (one instruction) rather
      // than shifting the digit again for a sign test.
      asm("" : "+v"(m[bit]));
      ones[bit] = __ballot(m[bit] != 0u);
    }
    // Lanes whose digit differs from this lane's in some bit: the OR over the
    // bits of (lanes with the bit set) ^ (this lane's bit), one v_bitop3_b32
    // per bit and half (truth table 0xF6: src0 | (src1 ^ src2)).
    uint32_t xlo = uint32_t(ones[0]) ^ m[0];
    uint32_t xhi = uint32_t(ones[0] >> 32) ^ m[0];
#pragma unroll
    for (int bit = 1; bit < BITS; ++bit) {
      xlo = __builtin_amdgcn_bitop3_b32(xlo, uint32_t(ones[bit]), m[bit], 0xF6);
      xhi = __builtin_amdgcn_bitop3_b32(xhi, uint32_t(ones[bit] >> 32), m[bit], 0xF6);
    }
    plo &= ~xlo;
    phi &= ~xhi;
    const uint32_t before = __builtin_amdgcn_mbcnt_hi(phi, __builtin_amdgcn_mbcnt_lo(plo, 0u));
    const uint32_t total = uint32_t(__popc(plo) + __popc(phi));
    uint32_t c = 0;
    if (FULL || valid) {
      c = wcnt[d];
      wcnt[d] = c + total;
    }
    rank[i] = c + before;
  }
}

// One stable LSD pass over BITS bits at `shift`: ticket -> load kTile / (64
// WAVES) elements per thread -> rank within each wave -> per-digit workgroup
// counts -> look-back for the global offsets -> reorder the tile in LDS by
// digit -> coalesced stores.
// vals_in == nullptr means vals[i] = i.
// With `remap` (the first pass of a remapped plan), the keys are mapped to
// min(key - base, cap) as they are loaded, and written so.  PAY: a second
// 32-bit value per element (pay_in, in the input order) moves with the keys
// to pay_out.
template <typename K, int BITS, bool PAY, int WAVES = 4>
__global__ __launch_bounds__(WAVES * 64) void scatter_kernel(
    const K* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, K* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out, int64_t n, int shift, const uint32_t* __restrict__ hist,
    uint64_t* __restrict__ status, uint32_t* __restrict__ ticket, uint32_t* __restrict__ err,
    const uint32_t* __restrict__ pay_in, uint32_t* __restrict__ pay_out, bool remap,
    uint64_t remap_base, uint64_t remap_cap) {
  constexpr int D = 1 << BITS;
  constexpr int kThreads = WAVES * 64;
  constexpr int ITEMS = kTile / kThreads;  // per thread
  static_assert(ITEMS * kThreads == kTile, "whole items per thread");
  static_assert(D <= kThreads || D % kThreads == 0, "digits per thread");
  // Per-digit work: DPT consecutive digits per thread (d = DPT t + q), so one
  // block scan orders them all.
  constexpr int DPT = D > kThreads ? D / kThreads : 1;
  constexpr int kSeg = kTile / WAVES;  // contiguous elements per wave
  __shared__ uint32_t cnt[WAVES][D];
  __shared__ uint32_t gofs[D];
  __shared__ uint32_t scratch[WAVES];
  __shared__ int s_block;
  __shared__ K skeys[kTile];
  __shared__ uint32_t svals[kTile];
  __shared__ uint32_t spay[PAY ? kTile : 1];

  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  if (threadIdx.x == 0) s_block = int(atomicAdd(ticket, 1u));
  for (int d = threadIdx.x; d < WAVES * D; d += kThreads) (&cnt[0][0])[d] = 0;
  __syncthreads();
  const int b = s_block;
  const int64_t base = int64_t(b) * kTile;
  const int nvalid = int(min(int64_t(kTile), n - base));
  const bool full = nvalid == kTile;
  const int seg_valid = nvalid - wid * kSeg;  // valid elements from this wave's segment start
  const K* kin = keys_in + base + wid * kSeg;

  K key[ITEMS];
  uint32_t val[ITEMS];
  uint32_t pay[PAY ? ITEMS : 1];
  uint32_t dig[ITEMS];
  if (full) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) key[i] = kin[i * 64 + lane];
    if constexpr (PAY) {
      const uint32_t* pin = pay_in + base + wid * kSeg;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) pay[i] = pin[i * 64 + lane];
    }
    if (vals_in) {
      const uint32_t* vin = vals_in + base + wid * kSeg;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) val[i] = vin[i * 64 + lane];
    } else {
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) val[i] = uint32_t(base) + uint32_t(wid * kSeg + i * 64 + lane);
    }
  } else {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int o = i * 64 + lane;
      const bool valid = o < seg_valid;
      key[i] = valid ? kin[o] : K(0);
      val[i] = valid ? (vals_in ? vals_in[base + wid * kSeg + o] : uint32_t(base + wid * kSeg + o))
                     : 0u;
      if constexpr (PAY) pay[i] = valid ? pay_in[base + wid * kSeg + o] : 0u;
    }
  }
  if (remap) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) key[i] = min(K(key[i] - K(remap_base)), K(remap_cap));
  }
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) dig[i] = uint32_t(key[i] >> shift) & (D - 1);

  uint32_t rank[ITEMS];
  if (full)
    rank_items<BITS, true, ITEMS>(dig, seg_valid, cnt[wid], rank);
  else
    rank_items<BITS, false, ITEMS>(dig, seg_valid, cnt[wid], rank);
  __syncthreads();

  // cw[q][w]: wave w's count of the thread's digit q.
  uint32_t tot[DPT], cw[DPT][WAVES], hv[DPT];
  uint32_t tsum = 0, hsum = 0;
#pragma unroll
  for (int q = 0; q < DPT; ++q) {
    const int d = DPT * int(threadIdx.x) + q;
    tot[q] = hv[q] = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      cw[q][w] = d < D ? cnt[w][d] : 0u;
      tot[q] += cw[q][w];
    }
    if (d < D) hv[q] = hist[d];
    tsum += tot[q];
    hsum += hv[q];
  }
  uint32_t all;
  uint32_t local_start = block_exclusive_scan_waves<WAVES>(tsum, scratch, all);
  uint32_t digit_base = block_exclusive_scan_waves<WAVES>(hsum, scratch, all);
  uint64_t excl[DPT];
#pragma unroll
  for (int q = 0; q < DPT; ++q) {
    const int d = DPT * int(threadIdx.x) + q;
    excl[q] = 0;
    if (d < D)
      store_status(status + int64_t(b) * D + d,
                   (b == 0 ? kFlagPrefix : kFlagAggregate) | uint64_t(tot[q]));
  }
#pragma unroll
  for (int q = 0; q < DPT; ++q) {
    const int d = DPT * int(threadIdx.x) + q;
    if (d < D) {
      // Wave w's items of digit d start at cnt[w][d] in the reordered tile.
      uint32_t start = local_start;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        cnt[w][d] = start;
        start += cw[q][w];
      }
      if (b > 0) {
        excl[q] = look_back(status, D, b, d, err);
        store_status(status + int64_t(b) * D + d, kFlagPrefix | (excl[q] + tot[q]));
      }
      // Output position of reordered item j of digit d: gofs[d] + j (mod 2^32).
      gofs[d] = digit_base + uint32_t(excl[q]) - local_start;
    }
    local_start += tot[q];
    digit_base += hv[q];
  }
  __syncthreads();

#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if (full || i * 64 + lane < seg_valid) {
      const uint32_t pos = cnt[wid][dig[i]] + rank[i];
      skeys[pos] = key[i];
      svals[pos] = val[i];
      if constexpr (PAY) spay[pos] = pay[i];
    }
  }
  __syncthreads();

  for (int j = threadIdx.x; j < nvalid; j += kThreads) {
    const K k = skeys[j];
    const uint32_t d = uint32_t(k >> shift) & (D - 1);
    const uint32_t o = gofs[d] + uint32_t(j);
    keys_out[o] = k;
    vals_out[o] = svals[j];
    if constexpr (PAY) pay_out[o] = spay[j];
  }
}

// value(i) = in[order ? order[i] : i], widened to Out.  load4 reads the four
// values at i (a multiple of 4) with one 16-byte load of `order` or `in`.
template <typename In, typename Out>
struct GatherLoad {
  const In* in;
  const int32_t* order;
  __device__ Out operator()(int64_t i) const { return Out(in[order ? order[i] : i]); }
  __device__ void load4(int64_t i, Out (&v)[4]) const {
    if (order) {
      const int4 o = *reinterpret_cast<const int4*>(order + i);
      v[0] = Out(in[o.x]);
      v[1] = Out(in[o.y]);
      v[2] = Out(in[o.z]);
      v[3] = Out(in[o.w]);
    } else {
      static_assert(sizeof(In) == 4, "vector path reads four 32-bit values");
      const int4 q = *reinterpret_cast<const int4*>(in + i);
      v[0] = Out(In(q.x));
      v[1] = Out(In(q.y));
      v[2] = Out(In(q.z));
      v[3] = Out(In(q.w));
    }
  }
};

__device__ __forceinline__ void store4(uint32_t* p, const uint32_t (&v)[4]) {
  *reinterpret_cast<uint4*>(p) = make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void store4(int64_t* p, const int64_t (&v)[4]) {
  reinterpret_cast<longlong2*>(p)[0] = make_longlong2(v[0], v[1]);
  reinterpret_cast<longlong2*>(p)[1] = make_longlong2(v[2], v[3]);
}

// Per-element hook of scan_kernel: sink.all(e, prefix, value, n) receives
// the thread's M elements e[m] (exclusive prefix and value each; elements at
// or past n are not real), so a sink's own reads can be issued together.
struct NoSink {
  template <int M, typename Out>
  __device__ void all(const int64_t (&)[M], const Out (&)[M], const Out (&)[M], int64_t) const {}
};

template <typename T>
__device__ __forceinline__ T from_lane63(T v) {
  if constexpr (sizeof(T) == 4) {
    return T(__builtin_amdgcn_readlane(int(v), 63));
  } else {
    return __shfl(v, 63, 64);
  }
}

// The row list's width scan runs as one look-back kernel up to this many
// tiles (short chains, one launch) and as reduce-then-scan beyond (three
// launches, no chain): config 3's 950 tiles 30 -> 23 us, config 4's 199 ->
// 138 us.  The height scan keeps the look-back: its tile sums gather through
// the depth order, which costs more than its chain (config 3 15 -> 24 us).
constexpr int64_t kLookBackScanTiles = 16;

// Loads the thread's 16 elements of tile b (the layout of scan_kernel).
template <typename Out, typename Load>
__device__ __forceinline__ void load_tile(const Load& load, int64_t n, bool vec, int64_t base,
                                          int wid, int lane, Out (&v)[4][4]) {
  // A full tile (the workgroup-uniform case) loads its four groups without
  // per-lane branches, so all of a thread's loads are in flight together.
  const bool full = vec && base + kTile <= n;
  if (full) {
#pragma unroll
    for (int i = 0; i < 4; ++i) load.load4(base + 4 * (wid * 256 + i * 64 + lane), v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t e = base + 4 * (wid * 256 + i * 64 + lane);
      if (vec && e + 4 <= n) {
        load.load4(e, v[i]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[i][j] = e + j < n ? load(e + j) : Out(0);
      }
    }
  }
}

// Reduce-then-scan, step 1: sums[b] = the sum of tile b's elements.
template <typename Out, typename Load>
__global__ __launch_bounds__(kBlock) void tile_sum_kernel(Load load, int64_t n, bool vec,
                                                          Out* __restrict__ sums) {
  __shared__ Out part[4];
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  Out v[4][4];
  load_tile<Out>(load, n, vec, int64_t(blockIdx.x) * kTile, wid, lane, v);
  Out t = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) t += v[i][0] + v[i][1] + v[i][2] + v[i][3];
  t = wave_sum(t);
  if (lane == 0) part[wid] = t;
  __syncthreads();
  if (threadIdx.x == 0) sums[blockIdx.x] = part[0] + part[1] + part[2] + part[3];
}

// Reduce-then-scan, step 2 (one workgroup): the tile sums become the tiles'
// exclusive offsets, in place; *total_out = the grand total when non-null.
// Each thread owns a contiguous run of tiles and issues its loads eight at a
// time.
template <typename Out>
__global__ __launch_bounds__(kBlock) void tile_offsets_kernel(Out* __restrict__ sums, int64_t nb,
                                                              Out* __restrict__ total_out) {
  __shared__ Out scratch[4];
  const int64_t per = (nb + kBlock - 1) / kBlock;
  const int64_t lo = int64_t(threadIdx.x) * per, hi = min(lo + per, nb);
  Out acc = 0;
  for (int64_t i = lo; i < hi; i += 8) {
    Out c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = i + j < hi ? sums[i + j] : Out(0);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += c[j];
  }
  Out total;
  Out run = block_exclusive_scan(acc, scratch, total);
  for (int64_t i = lo; i < hi; i += 8) {
    Out c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = i + j < hi ? sums[i + j] : Out(0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (i + j < hi) {
        sums[i + j] = run;
        run += c[j];
      }
    }
  }
  if (threadIdx.x == 0 && total_out) *total_out = total;
}

// Exclusive scan of load(i) into out[0..n), and out[n] = total when
// write_total; kTile elements per workgroup.  With `offsets` (the tiles'
// exclusive offsets from tile_sum_kernel + tile_offsets_kernel) the
// workgroups need no ticket and no look-back; otherwise one kernel.  Accesses are fully
// coalesced: lane l of wave w handles the four-element groups
// w * 256 + i * 64 + l (i < 4) of the tile, read and written with 16-byte
// accesses when `vec` (load.load4 and out are 16-byte aligned); four wave
// scans order the groups, one LDS exchange orders the waves, and a wave-wide
// look-back gives the tile's offset.  sink.all sees every element with
// out[i] and its value.
template <typename Out, typename Load, typename Sink = NoSink>
__global__ __launch_bounds__(kBlock) void scan_kernel(Load load, int64_t n, Out* __restrict__ out,
                                                      bool write_total, bool vec,
                                                      uint64_t* __restrict__ status,
                                                      uint32_t* __restrict__ ticket,
                                                      uint32_t* __restrict__ err,
                                                      Sink sink = Sink{},
                                                      const Out* __restrict__ offsets = nullptr) {
  static_assert(kTile == 4 * 4 * kBlock, "16 elements per thread in groups of four");
  __shared__ Out wave_total[4];
  __shared__ Out s_excl;
  __shared__ int s_block;
  if (!offsets) {
    if (threadIdx.x == 0) s_block = int(atomicAdd(ticket, 1u));
    __syncthreads();
  }
  const int b = offsets ? int(blockIdx.x) : s_block;
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int64_t base = int64_t(b) * kTile;
  Out v[4][4];
  Out group_sum[4];
  load_tile<Out>(load, n, vec, base, wid, lane, v);
#pragma unroll
  for (int i = 0; i < 4; ++i) group_sum[i] = v[i][0] + v[i][1] + v[i][2] + v[i][3];
  // Exclusive prefix of each group inside the wave's 1024 elements.
  Out carry = 0;
  Out group_pre[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const Out inc = wave_inclusive_scan(group_sum[i]);
    group_pre[i] = carry + inc - group_sum[i];
    carry += from_lane63(inc);
  }
  if (lane == 0) wave_total[wid] = carry;
  __syncthreads();
  Out before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const Out t = wave_total[w];
    if (w < wid) before += t;
    total += t;
  }
  if (offsets) {
    if (threadIdx.x == 0) s_excl = offsets[b];
  } else if (threadIdx.x < 64) {
    if (threadIdx.x == 0)
      store_status(status + b, (b == 0 ? kFlagPrefix : kFlagAggregate) | uint64_t(total));
    const uint64_t excl = b > 0 ? wave_look_back(status, b, err) : 0;
    if (threadIdx.x == 0) {
      if (b > 0) store_status(status + b, kFlagPrefix | (excl + uint64_t(total)));
      s_excl = Out(excl);
      if (write_total && b == int(gridDim.x) - 1) out[n] = Out(excl) + total;
    }
  }
  __syncthreads();
  const Out offset = s_excl + before;
  int64_t es[16];
  Out rs[16], vs[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t e = base + 4 * (wid * 256 + i * 64 + lane);
    Out r[4];
    r[0] = offset + group_pre[i];
    r[1] = r[0] + v[i][0];
    r[2] = r[1] + v[i][1];
    r[3] = r[2] + v[i][2];
    if (vec && e + 4 <= n) {
      store4(out + e, r);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (e + j < n) out[e + j] = r[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      es[4 * i + j] = e + j;
      rs[4 * i + j] = r[j];
      vs[4 * i + j] = v[i][j];
    }
  }
  sink.all(es, rs, vs, n);
}

}  // namespace sweep
}  // namespace gs
