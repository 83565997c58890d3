// C-ABI bookkeeping: per-thread error text, version, argument validation,
// the side streams used to overlap independent stages, and the per-device
// word of device-side check failures.
#include <cstdarg>
#include <cstdio>
#include <mutex>

#include <algorithm>

#include "common.h"

namespace gs {

namespace {
thread_local char g_error[512] = {0};
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = 0; }

namespace {
thread_local LaunchEvents g_launch_events;
thread_local bool g_launch_events_taken = false;
}  // namespace

LaunchEvents take_launch_events() {
  const LaunchEvents e = g_launch_events;
  if (e.start || e.stop) g_launch_events_taken = true;
  g_launch_events = LaunchEvents{};
  return e;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: HIP launch failed: %s", what, hipGetErrorString(err));
    return GS_ERR_HIP;
  }
  return GS_OK;
}

int check_view(const gs_view& v, bool need_tiles) {
  GS_REQUIRE(v.image_width > 0 && v.image_height > 0, GS_ERR_INVALID_ARGUMENT,
             "image size must be positive, got %dx%d", v.image_width, v.image_height);
  GS_REQUIRE(v.rendering_mode == GS_MODE_GAUSSIAN || v.rendering_mode == GS_MODE_ELLIPSOID,
             GS_ERR_INVALID_ARGUMENT, "unknown rendering mode %d", v.rendering_mode);
  if (need_tiles) {
    GS_REQUIRE(is_pow2(v.tile_size), GS_ERR_INVALID_ARGUMENT,
               "tile_size must be a positive power of two, got %d", v.tile_size);
    GS_REQUIRE(v.tile_size >= 4 && v.tile_size <= 32, GS_ERR_UNSUPPORTED,
               "tile_size %d not supported (4, 8, 16 or 32)", v.tile_size);
    GS_REQUIRE(v.views >= 0 && v.mosaic_cols >= 0 && v.active_tiles >= 0,
               GS_ERR_INVALID_ARGUMENT, "views, mosaic_cols and active_tiles must be non-negative");
    const int views = v.views > 1 ? v.views : 1;
    const int cols = std::min(views, v.mosaic_cols > 1 ? v.mosaic_cols : 1);
    const int64_t rows = (views + cols - 1) / cols;
    const int64_t tiles = int64_t(tiles_along(v.image_width, v.tile_size)) * cols *
                          tiles_along(v.image_height, v.tile_size) * rows;
    GS_REQUIRE(tiles < (int64_t(1) << 30), GS_ERR_OVERFLOW, "too many tiles (%lld)",
               (long long)tiles);
    GS_REQUIRE(int64_t(v.image_width) * v.image_height * views < (int64_t(1) << 40),
               GS_ERR_OVERFLOW, "too many pixels");
  }
  return GS_OK;
}

namespace {
constexpr int kMaxDevices = 64;
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr;
  hipEvent_t join = nullptr;
};
// Per thread: a thread's fork-to-join sequence uses its own stream and
// events, so no lock is held across the host wait of a join (threads that
// end leave their streams to the process's end).
thread_local SideStream g_side[kMaxDevices];
}  // namespace

int stream_device(hipStream_t stream, int* device) {
  if (stream) {
    GS_REQUIRE(hipStreamGetDevice(stream, device) == hipSuccess, GS_ERR_HIP,
               "hipStreamGetDevice failed");
  } else {
    GS_REQUIRE(hipGetDevice(device) == hipSuccess, GS_ERR_HIP, "hipGetDevice failed");
  }
  GS_REQUIRE(*device >= 0 && *device < kMaxDevices, GS_ERR_HIP, "device %d out of range", *device);
  return GS_OK;
}

int fork_side_stream(hipStream_t main, SideFork& f) {
  int device = 0;
  GS_TRY(stream_device(main, &device));
  SideStream& s = g_side[device];
  if (!s.stream) {
    int current = 0;
    GS_REQUIRE(hipGetDevice(&current) == hipSuccess, GS_ERR_HIP, "hipGetDevice failed");
    const bool switch_device = current != device;
    if (switch_device) GS_REQUIRE(hipSetDevice(device) == hipSuccess, GS_ERR_HIP, "hipSetDevice");
    // Default priority; the stream does not synchronise with the null stream.
    const bool ok = hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking) == hipSuccess &&
                    hipEventCreateWithFlags(&s.fork, hipEventDisableTiming) == hipSuccess &&
                    hipEventCreateWithFlags(&s.join, hipEventDisableTiming) == hipSuccess;
    if (switch_device) (void)hipSetDevice(current);
    GS_REQUIRE(ok, GS_ERR_HIP, "could not create the side stream");
  }
  GS_REQUIRE(hipEventRecord(s.fork, main) == hipSuccess &&
                 hipStreamWaitEvent(s.stream, s.fork, 0) == hipSuccess,
             GS_ERR_HIP, "side stream fork failed");
  f.main = main;
  f.side = s.stream;
  f.join = s.join;
  return GS_OK;
}

int join_side_stream(SideFork& f, bool host_wait) {
  bool ok = hipEventRecord(f.join, f.side) == hipSuccess;
  // With the host's wait, work the caller enqueues after this call follows
  // the side stream's: the caller's stream is not given a wait packet (each
  // one delays its next kernel by a few microseconds).
  if (ok) ok = host_wait ? hipEventSynchronize(f.join) == hipSuccess
                         : hipStreamWaitEvent(f.main, f.join, 0) == hipSuccess;
  GS_REQUIRE(ok, GS_ERR_HIP, "side stream join failed");
  return GS_OK;
}

// Sticky word of device-side check failures (kDeviceFlag* bits), one copy
// per GPU.  Kernels receive its address (device_flags) and set bits with a
// global atomic OR; the host reads it with gs_device_errors or through the
// fifth word gs_bin_tiles_plan copies beside its totals.
static __device__ __align__(16) uint32_t g_device_flags[4];
namespace {
uint32_t* g_flags_addr[kMaxDevices] = {};
std::mutex g_flags_mutex;
}  // namespace

int device_flags(hipStream_t stream, uint32_t** flags) {
  int device = 0;
  GS_TRY(stream_device(stream, &device));
  std::lock_guard<std::mutex> lock(g_flags_mutex);
  if (!g_flags_addr[device]) {
    // Each GPU holds its own copy of the array at its own address: look it up
    // with that device current.
    int current = 0;
    GS_REQUIRE(hipGetDevice(&current) == hipSuccess, GS_ERR_HIP, "hipGetDevice failed");
    const bool switch_device = current != device;
    if (switch_device) GS_REQUIRE(hipSetDevice(device) == hipSuccess, GS_ERR_HIP, "hipSetDevice");
    void* addr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(g_device_flags));
    if (switch_device) (void)hipSetDevice(current);
    GS_REQUIRE(e == hipSuccess && addr, GS_ERR_HIP, "device flags lookup failed: %s",
               hipGetErrorString(e));
    g_flags_addr[device] = static_cast<uint32_t*>(addr);
  }
  *flags = g_flags_addr[device];
  return GS_OK;
}

}  // namespace gs

extern "C" {

GS_API int gs_device_errors(uint32_t* flags, int32_t clear, void* stream) {
  using namespace gs;
  clear_error();
  GS_REQUIRE(flags, GS_ERR_INVALID_ARGUMENT, "null pointer argument");
  hipStream_t s = as_stream(stream);
  uint32_t* dev = nullptr;
  GS_TRY(device_flags(s, &dev));
  // Synchronous by design: the caller asks for the state after its work.
  GS_REQUIRE(hipMemcpyAsync(flags, dev, sizeof(uint32_t), hipMemcpyDeviceToHost, s) == hipSuccess &&
                 hipStreamSynchronize(s) == hipSuccess,
             GS_ERR_HIP, "device_errors: read failed");
  if (clear && *flags) {
    const uint32_t zero = 0;
    GS_REQUIRE(hipMemcpyAsync(dev, &zero, sizeof(uint32_t), hipMemcpyHostToDevice, s) ==
                       hipSuccess &&
                   hipStreamSynchronize(s) == hipSuccess,
               GS_ERR_HIP, "device_errors: clear failed");
  }
  return GS_OK;
}

GS_API int gs_abi_version(void) { return GS_ABI_VERSION; }

GS_API int gs_arm_launch_events(void* start, void* stop) {
  gs::clear_error();
  gs::g_launch_events = gs::LaunchEvents{static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)};
  gs::g_launch_events_taken = false;
  return GS_OK;
}

GS_API int gs_disarm_launch_events(void) {
  const int taken = gs::g_launch_events_taken ? 1 : 0;
  gs::g_launch_events = gs::LaunchEvents{};
  gs::g_launch_events_taken = false;
  return taken;
}

GS_API const char* gs_last_error(void) { return gs::g_error; }

}  // extern "C"
