// C-ABI bookkeeping: per-thread error text, version, argument validation.
#include <cstdarg>
#include <cstdio>

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
    const int64_t tiles = int64_t(tiles_along(v.image_width, v.tile_size)) *
                          tiles_along(v.image_height, v.tile_size);
    GS_REQUIRE(tiles < (int64_t(1) << 30), GS_ERR_OVERFLOW, "too many tiles (%lld)",
               (long long)tiles);
  }
  return GS_OK;
}

}  // namespace gs

extern "C" {

GS_API int gs_abi_version(void) { return GS_ABI_VERSION; }

GS_API const char* gs_last_error(void) { return gs::g_error; }

}  // extern "C"
