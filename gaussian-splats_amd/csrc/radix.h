// Host-side drivers of the onesweep kernels shared by the binning paths:
// scratch layout, the LSD radix sort and the look-back scan.
#pragma once

#include <algorithm>

#include "common.h"
#include "onesweep.h"

namespace gs {

using sweep::kTile;
using sweep::kBlock;

inline int bits_for(int64_t count) {  // ceil(log2(count)), 0 for count <= 1
  int b = 0;
  while ((int64_t(1) << b) < count) ++b;
  return b;
}

// Scratch shared by the sort and the scan: ping-pong buffers, then one zeroed
// region (look-back status words of every sort pass and of the scan, then the
// 32-bit histograms and tickets).  Check failures go to the device's sticky
// flags word (`flags`, set by the caller from device_flags).
struct Scratch {
  void* keys_alt = nullptr;
  uint32_t* vbuf[2] = {nullptr, nullptr};
  uint32_t* pbuf[2] = {nullptr, nullptr};  // payload ping-pong (carved with `payload`)
  uint64_t* sort_status = nullptr;
  uint64_t* scan_status = nullptr;
  uint64_t* zero_begin = nullptr;
  int64_t zero_words = 0;  // 64-bit words of status
  uint32_t* small = nullptr;  // hist[kMaxPasses*kHistStride], tickets[kMaxPasses], scan ticket
  int small_words = 0;
  size_t bytes = 0;
  uint32_t* flags = nullptr;  // the device's sticky check-failure word

  uint32_t* hist() const { return small; }
  uint32_t* tickets() const { return small + sweep::kMaxPasses * sweep::kHistStride; }
  uint32_t* scan_ticket() const { return tickets() + sweep::kMaxPasses; }
};

inline int64_t sort_status_words(int64_t n, const sweep::Plan& p) {
  const int64_t nblocks = ceil_div(n, kTile);
  int64_t words = 0;
  for (int i = 0; i < p.passes; ++i) words += nblocks << p.bits[i];
  return words;
}

// Lays out scratch for a sort of n keys of key_bytes over at most end_bit
// bits in digits of at most max_bits (end_bit < 0: no sort) and a scan of
// scan_n elements (0: no scan).  The look-back statuses are sized for the
// largest plan of any end bit up to end_bit.
inline Scratch carve(void* ws, int64_t n, int key_bytes, int end_bit, int64_t scan_n,
                     int max_bits = 8, bool payload = false) {
  Scratch s;
  char* p = static_cast<char*>(ws);
  size_t off = 0;
  int64_t sort_words = 0;
  if (end_bit >= 0 && n > 0) {
    s.keys_alt = p ? p + off : nullptr;
    off += align_up(size_t(n) * key_bytes);
    for (int i = 0; i < 2; ++i) {
      s.vbuf[i] = p ? reinterpret_cast<uint32_t*>(p + off) : nullptr;
      off += align_up(size_t(n) * 4);
    }
    for (int i = 0; payload && i < 2; ++i) {
      s.pbuf[i] = p ? reinterpret_cast<uint32_t*>(p + off) : nullptr;
      off += align_up(size_t(n) * 4);
    }
    for (int e = 1; e <= end_bit; ++e)
      sort_words = std::max(sort_words, sort_status_words(n, sweep::make_plan(e, max_bits)));
  }
  const int64_t scan_words = scan_n > 0 ? ceil_div(scan_n, kTile) : 0;
  s.zero_begin = p ? reinterpret_cast<uint64_t*>(p + off) : nullptr;
  s.sort_status = s.zero_begin;
  s.scan_status = p ? s.zero_begin + sort_words : nullptr;
  s.zero_words = sort_words + scan_words;
  off += align_up(size_t(s.zero_words) * 8);
  s.small_words = sweep::kMaxPasses * sweep::kHistStride + sweep::kMaxPasses + 1;
  s.small = p ? reinterpret_cast<uint32_t*>(p + off) : nullptr;
  off += align_up(size_t(s.small_words) * 4);
  s.bytes = off;
  return s;
}

inline void clear(const Scratch& s, hipStream_t stream) {
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(1024, ceil_div(s.zero_words, kBlock)));
  sweep::clear_kernel<<<unsigned(blocks), kBlock, 0, stream>>>(s.zero_begin, s.zero_words, s.small,
                                                               s.small_words);
}

// Waves per workgroup of the scatter passes (kTile / (64 kScatterWaves) keys
// per thread).  Eight waves of 8 keys, two per SIMD, hide more of a pass's
// dependent steps than four waves of 16 (82 VGPRs instead of 145): depth sort
// passes on 1M keys 19.4 -> 18.2 us (7-bit digits), 17.6 -> 16.1 (6-bit), on
// 4M keys 50.8 -> 49.7 and 41.6 -> 37.9; on 8M keys the 7-bit passes are
// slower (75 -> 80 us) and the 6-bit one faster (108 -> 98).
constexpr int kScatterWaves = 8;

template <typename K, int BITS>
void launch_scatter(const K* kin, const uint32_t* vin, K* kout, uint32_t* vout, int64_t n,
                    int shift, const uint32_t* hist, uint64_t* status, uint32_t* ticket,
                    uint32_t* err, const uint32_t* pin, uint32_t* pout, bool remap,
                    uint64_t base, uint64_t cap, hipStream_t s) {
  const unsigned nblocks = unsigned(ceil_div(n, kTile));
  constexpr int W = kScatterWaves;
  if (pin)
    sweep::scatter_kernel<K, BITS, true, W><<<nblocks, W * 64, 0, s>>>(
        kin, vin, kout, vout, n, shift, hist, status, ticket, err, pin, pout, remap, base, cap);
  else
    sweep::scatter_kernel<K, BITS, false, W><<<nblocks, W * 64, 0, s>>>(
        kin, vin, kout, vout, n, shift, hist, status, ticket, err, nullptr, nullptr, remap, base,
        cap);
}

template <typename K>
void dispatch_scatter(int bits, const K* kin, const uint32_t* vin, K* kout, uint32_t* vout,
                      int64_t n, int shift, const uint32_t* hist, uint64_t* status,
                      uint32_t* ticket, uint32_t* err, const uint32_t* gsrc, uint32_t* gout,
                      bool remap, uint64_t base, uint64_t cap, hipStream_t s) {
  // One launch per digit width (the kernel's template argument).
#define GS_SCATTER(B)                                                                  \
  launch_scatter<K, B>(kin, vin, kout, vout, n, shift, hist, status, ticket, err, gsrc, gout, \
                       remap, base, cap, s)
  switch (bits) {
    case 1: GS_SCATTER(1); break;
    case 2: GS_SCATTER(2); break;
    case 3: GS_SCATTER(3); break;
    case 4: GS_SCATTER(4); break;
    case 5: GS_SCATTER(5); break;
    case 6: GS_SCATTER(6); break;
    case 7: GS_SCATTER(7); break;
    default: GS_SCATTER(8); break;
  }
#undef GS_SCATTER
}

// Sorts (keys, vals) on bits [0, end_bit) after `clear` has zeroed the scratch.
// vals == nullptr means vals[i] = i.  Sorted values land in vals_final;
// *keys_final points at the sorted keys (keys or the scratch copy).
// SPREAD: the keys are depth keys (see hist_kernel).  payload_src (optional,
// with scratch carved with `payload`): a second value per element, in the
// input order, that moves with the keys to payload_final.
// hook() is called on the host once the histogram and the first pass are
// enqueued, before the other passes (it may enqueue work on another stream):
// the caller's stream has those two kernels to run while the host enqueues
// it.
struct NoHook {
  int operator()() const { return GS_OK; }
};
// KeyRemap: sort min(key - base, 2^end_bit - 1) (the scratch was carved for
// `max_bits`); keys below base or at least base + 2^end_bit - 1 sort last,
// in index order.  Off: the keys' bits [0, end_bit) in digits of at most 8
// bits.
struct KeyRemap {
  bool on = false;
  uint64_t base = 0;
  int max_bits = 8;
};
template <typename K, bool SPREAD = false, typename Hook = NoHook>
int radix_sort(K* keys, const uint32_t* vals, int64_t n, int end_bit, uint32_t* vals_final,
               K** keys_final, const Scratch& ws, hipStream_t s,
               const uint32_t* payload_src = nullptr, uint32_t* payload_final = nullptr,
               Hook hook = Hook{}, KeyRemap remap = KeyRemap{}) {
  GS_REQUIRE(n < (int64_t(1) << 32) - kTile, GS_ERR_OVERFLOW, "too many elements to sort (%lld)",
             (long long)n);
  GS_REQUIRE(end_bit <= int(8 * sizeof(K)), GS_ERR_INVALID_ARGUMENT,
             "end bit %d beyond the %d-bit key", end_bit, int(8 * sizeof(K)));
  *keys_final = keys;
  if (n == 0) return hook();
  GS_REQUIRE(remap.max_bits >= 1 && remap.max_bits <= sweep::kMaxDigitBits &&
                 (!remap.on || end_bit < int(8 * sizeof(K))),
             GS_ERR_INVALID_ARGUMENT, "bad key remap (%d-bit digits, end bit %d)", remap.max_bits,
             end_bit);
  sweep::Plan plan = sweep::make_plan(end_bit, remap.max_bits);
  plan.remap = remap.on;
  plan.base = remap.base;
  plan.cap = remap.on ? (uint64_t(1) << end_bit) - 1 : ~uint64_t(0);
  const int hist_blocks =
      int(std::min<int64_t>(1024, ceil_div(n, sweep::kHistBlock * sweep::kHistKeys)));
  sweep::hist_kernel<K, SPREAD>
      <<<unsigned(hist_blocks), sweep::kHistBlock, 0, s>>>(keys, n, plan, ws.hist());
  GS_REQUIRE(!payload_src || (payload_final && ws.pbuf[0] && ws.pbuf[1]),
             GS_ERR_INVALID_ARGUMENT, "payload without its buffers");
  K* kbuf[2] = {static_cast<K*>(ws.keys_alt), keys};
  const K* kin = keys;
  const uint32_t* vin = vals;
  const uint32_t* pin = payload_src;
  uint64_t* status = ws.sort_status;
  const int64_t nblocks = ceil_div(n, kTile);
  for (int pass = 0; pass < plan.passes; ++pass) {
    K* kout = kbuf[pass & 1];
    const bool last = pass == plan.passes - 1;
    uint32_t* vout = last ? vals_final : ws.vbuf[pass & 1];
    uint32_t* pout = pin ? (last ? payload_final : ws.pbuf[pass & 1]) : nullptr;
    dispatch_scatter<K>(plan.bits[pass], kin, vin, kout, vout, n, plan.shift[pass],
                        ws.hist() + pass * sweep::kHistStride, status, ws.tickets() + pass,
                        ws.flags, pin, pout, pass == 0 && plan.remap, plan.base, plan.cap, s);
    status += nblocks << plan.bits[pass];
    kin = kout;
    vin = vout;
    pin = pout;
    if (pass == 0) GS_TRY(hook());
  }
  *keys_final = const_cast<K*>(kin);
  return check_launch("radix_sort");
}

// `vec`: the loader's 16-byte reads and `out` are 16-byte aligned.
template <typename Out, typename Load, typename Sink = sweep::NoSink>
void launch_scan(Load load, int64_t n, Out* out, bool write_total, bool vec, const Scratch& ws,
                 hipStream_t s, Sink sink = Sink{}) {
  vec = vec && (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
  sweep::scan_kernel<Out, Load, Sink><<<unsigned(ceil_div(n, kTile)), sweep::kBlock, 0, s>>>(
      load, n, out, write_total, vec, ws.scan_status, ws.scan_ticket(), ws.flags, sink);
}

inline bool aligned_16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename T>
__global__ void fill_kernel(T* p, int64_t n, T value) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = value;
}

}  // namespace gs
