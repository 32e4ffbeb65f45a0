// Shared host/device helpers for the gfx950 Gabor rasterizer library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>

#include "gabor_hip.h"

namespace gs {

constexpr int kTile = 16;          // tile edge in pixels
constexpr int kTilePixels = 256;   // one workgroup of four wave64s per tile
constexpr int kGeometry = 17;      // floats per projected pair record
constexpr int kMaps = 9;           // output channels per pixel
constexpr int kClassic = 18;       // classic appearance floats per row
constexpr int kNeural = 57;        // neural appearance floats per row

// Thread-local error message surfaced through gs_last_error().
void set_error(const char* fmt, ...);
void clear_error();

// Map a HIP status to GS_ERR_HIP with a message; returns GS_OK on success.
int hip_status(hipError_t err, const char* what);

// Check the most recent launch on this thread.
int launch_status(const char* kernel);

// Event timing of kernel families (see gs_profile_enable).
struct ProfileScope {
  ProfileScope(int family, hipStream_t stream);
  ~ProfileScope();
  int family_;
  hipStream_t stream_;
  hipEvent_t start_ = nullptr;
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Tile grid of an image: ceil(W/16) x ceil(H/16).
inline int tiles_x(int width) { return (width + kTile - 1) / kTile; }
inline int tiles_y(int height) { return (height + kTile - 1) / kTile; }

}  // namespace gs

#define GS_REQUIRE(cond, code, ...)  \
  do {                               \
    if (!(cond)) {                   \
      ::gs::set_error(__VA_ARGS__);  \
      return (code);                 \
    }                                \
  } while (0)

#define GS_HIP(call)                                   \
  do {                                                 \
    int gs_status_ = ::gs::hip_status((call), #call);  \
    if (gs_status_ != GS_OK) return gs_status_;        \
  } while (0)

#define GS_LAUNCHED(name)                              \
  do {                                                 \
    int gs_status_ = ::gs::launch_status(name);        \
    if (gs_status_ != GS_OK) return gs_status_;        \
  } while (0)
