// Kernel 2: visible-pair packing and tile binning, plus kernel 3's range
// extraction.
//
// Tile rectangles use exactly the reference's float32 expressions
// (src/gabor_splatting/csrc/rasterize.cu:24-30):
//   x0 = int((x - r) / 16), x1 = int(((x + r) + 16 - 1) / 16), clamped to
//   [0, tw] (and y likewise), evaluated left to right in float32,
// so keys and ranges are bit-identical to the reference's for the same
// geometry and radii. Counts are computed on the fly inside the scan
// (never stored).
//
// Two binning pipelines give the same point list and ranges:
//  * reference order (gs_emit_tiles, gs_sort_pairs, gs_find_ranges): every
//    pair emits one 64-bit (image|tile) << 32 | depth-bits key per covered
//    tile, and the M keys are radix-sorted on 32 + bits(tiles) bits;
//  * depth first (gs_bin_order, then gs_bin_tiles), used by the renderer:
//    the Q pairs are stably sorted on their 32 depth bits, each pair then
//    emits its tiles in that order as 32-bit tile ids, and a stable sort on
//    only bits(tiles) bits groups them by tile. The first stage needs no
//    intersection count; M and V are summed by its first kernels, so the
//    host reads them while the depth sort runs. A stable sort of depth-ordered entries by tile
//    leaves each tile's entries ordered by (depth bits, pair index) - the
//    order of the 64-bit sort - while the M entries move through two 8-bit
//    passes of 8 bytes instead of 5-6 passes of 12 bytes.
#include <climits>

#include "common.hpp"
#include "index_guard.hpp"
#include "scan.hpp"
#include "sort.hpp"

namespace gs {
namespace {

// C++ int(float) on the reference's hardware truncates and saturates;
// the explicit form keeps that behaviour defined for any input.
__device__ __forceinline__ int trunc_to_int(float v) {
  if (v != v) return 0;
  if (v >= 2147483648.f) return INT_MAX;
  if (v <= -2147483648.f) return INT_MIN;
  return int(v);
}

struct TileRect {
  int x0, y0, x1, y1;
};

__device__ __forceinline__ TileRect tile_rect(float cx, float cy, int radius, int tw, int th) {
  const float r = float(radius);
  TileRect t;
  t.x0 = max(0, min(tw, trunc_to_int((cx - r) / 16.f)));
  t.y0 = max(0, min(th, trunc_to_int((cy - r) / 16.f)));
  t.x1 = max(0, min(tw, trunc_to_int((((cx + r) + 16.f) - 1.f) / 16.f)));
  t.y1 = max(0, min(th, trunc_to_int((((cy + r) + 16.f) - 1.f) / 16.f)));
  return t;
}

struct TileCountLoad {
  const float* geometry;
  const int* radii;
  int tw, th;
  __device__ int64_t operator()(int64_t i) const {
    const int r = radii[i];
    if (r <= 0) return 0;
    const TileRect t = tile_rect(geometry[i * kGeometry + 9], geometry[i * kGeometry + 10], r, tw, th);
    return int64_t(t.x1 - t.x0) * int64_t(t.y1 - t.y0);
  }
};

struct InclusiveStore {
  int64_t* out;
  __device__ void operator()(int64_t i, int64_t inclusive, int64_t) const { out[i] = inclusive; }
};

struct VisibleLoad {
  const int* radii;
  __device__ int64_t operator()(int64_t i) const { return radii[i] > 0 ? 1 : 0; }
};

struct SelectStore {
  int64_t* selected;
  int* row_of_pair;  // optional inverse map: row of pair i, or -1
  int64_t* num_selected;
  int64_t count;
  __device__ void operator()(int64_t i, int64_t inclusive, int64_t flag) const {
    if (flag) selected[inclusive - 1] = i;
    if (row_of_pair) row_of_pair[i] = flag ? int(inclusive - 1) : -1;
    if (i == count - 1) *num_selected = inclusive;
  }
};

__global__ __launch_bounds__(256) void zero_count_kernel(int64_t* value) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *value = 0;
}

__global__ __launch_bounds__(256) void emit_tiles_kernel(
    int64_t count, int tw, int th, const float* __restrict__ geometry,
    const int* __restrict__ radii, const int64_t* __restrict__ image_ids,
    const int64_t* __restrict__ offsets, uint64_t* __restrict__ keys,
    int* __restrict__ values) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= count) return;
  const int r = radii[i];
  if (r <= 0) return;
  const float* g = geometry + i * kGeometry;
  const TileRect t = tile_rect(g[9], g[10], r, tw, th);
  int64_t out = i == 0 ? 0 : offsets[i - 1];
  const uint64_t image_base = uint64_t(image_ids[i]) * uint64_t(tw) * uint64_t(th);
  const uint64_t depth_bits = __float_as_uint(g[8]);
  for (int y = t.y0; y < t.y1; ++y)
    for (int x = t.x0; x < t.x1; ++x) {
      const uint64_t tile = image_base + uint64_t(y * tw + x);
      keys[out] = (tile << 32) | depth_bits;
      values[out] = int(i);
      ++out;
    }
}

__global__ __launch_bounds__(64) void clear_flag_kernel(uint32_t* flag) {
  if (threadIdx.x == 0) *flag = 0u;
}

__global__ __launch_bounds__(256) void fill_ranges_kernel(int64_t tiles, int2* __restrict__ ranges) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < tiles) ranges[i] = make_int2(0, 0);
}

// Keys whose tile id lies outside [0, tiles) are ignored rather than
// written out of bounds.
__global__ __launch_bounds__(256) void find_ranges_kernel(int64_t m, int64_t tiles,
                                                          const uint64_t* __restrict__ keys,
                                                          int2* __restrict__ ranges) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= m) return;
  const uint64_t tile = keys[i] >> 32;
  const bool own = tile < uint64_t(tiles);
  if (i == 0) {
    if (own) ranges[tile].x = 0;
  } else {
    const uint64_t previous = keys[i - 1] >> 32;
    if (tile != previous) {
      if (previous < uint64_t(tiles)) ranges[previous].y = int(i);
      if (own) ranges[tile].x = int(i);
    }
  }
  if (i == m - 1 && own) ranges[tile].y = int(m);
}

// Depth-first binning, stage 1, step 1: each pair's tile rectangle
// (x0, y0, width, first tile id of its image) for stage 2, its tile count
// (the rectangle area of countTiles) and its depth key; pairs without
// tiles sort last. Each workgroup also stores its sums of the counts and of
// the pairs with tiles in partials[block], which totals_kernel adds up into
// M and V, so the host can read them before the pairs are sorted (plain
// stores and one more launch: thousands of workgroups adding into one
// device word would queue their atomics behind each other).
__global__ __launch_bounds__(256) void pair_keys_kernel(int64_t count, int tw, int th,
                                                        const float* __restrict__ geometry,
                                                        const int* __restrict__ radii,
                                                        const int64_t* __restrict__ image_ids,
                                                        uint32_t* __restrict__ keys,
                                                        int* __restrict__ values,
                                                        int* __restrict__ counts,
                                                        int4* __restrict__ rects,
                                                        long long* __restrict__ partials) {
  __shared__ long long wave_sums[2][4];
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  int c = 0;
  if (i < count) {
    const int r = radii[i];
    uint32_t key = 0xffffffffu;
    int4 rect = make_int4(0, 0, 1, 0);
    if (r > 0) {
      const float* g = geometry + i * kGeometry;
      const TileRect t = tile_rect(g[9], g[10], r, tw, th);
      c = (t.x1 - t.x0) * (t.y1 - t.y0);
      if (c > 0) {
        key = __float_as_uint(g[8]);
        rect = make_int4(t.x0, t.y0, t.x1 - t.x0, int(image_ids[i] * int64_t(tw) * th));
      }
    }
    counts[i] = c;
    keys[i] = key;
    values[i] = int(i);
    rects[i] = rect;
  }
  // Workgroup totals: wave sums by shuffles, then across the four waves.
  long long sum = c, with_tiles = c > 0 ? 1 : 0;
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    sum += __shfl_xor(sum, offset, 64);
    with_tiles += __shfl_xor(with_tiles, offset, 64);
  }
  const int wave = threadIdx.x >> 6;
  if (__lane_id() == 0) {
    wave_sums[0][wave] = sum;
    wave_sums[1][wave] = with_tiles;
  }
  __syncthreads();
  if (threadIdx.x < 2)
    partials[2 * int64_t(blockIdx.x) + threadIdx.x] =
        wave_sums[threadIdx.x][0] + wave_sums[threadIdx.x][1] + wave_sums[threadIdx.x][2] +
        wave_sums[threadIdx.x][3];
}

// M and V from pair_keys_kernel's `blocks` workgroup totals (one
// workgroup; `visible` may be null).
constexpr int kTotalsBlock = 1024;
__global__ __launch_bounds__(kTotalsBlock) void totals_kernel(const long long* __restrict__ partials,
                                                             int64_t blocks, int64_t* total,
                                                             int64_t* visible) {
  __shared__ long long wave_sums[2][kTotalsBlock / 64];
  long long sum = 0, with_tiles = 0;
  for (int64_t b = threadIdx.x; b < blocks; b += kTotalsBlock) {
    sum += partials[2 * b];
    with_tiles += partials[2 * b + 1];
  }
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    sum += __shfl_xor(sum, offset, 64);
    with_tiles += __shfl_xor(with_tiles, offset, 64);
  }
  if (__lane_id() == 0) {
    wave_sums[0][threadIdx.x >> 6] = sum;
    wave_sums[1][threadIdx.x >> 6] = with_tiles;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    long long value = 0;
#pragma unroll
    for (int w = 0; w < kTotalsBlock / 64; ++w) value += wave_sums[threadIdx.x][w];
    int64_t* target = threadIdx.x == 0 ? total : visible;
    if (target) *target = value;
  }
}

// No pairs: M = V = 0.
__global__ __launch_bounds__(64) void zero_totals_kernel(int64_t* total, int64_t* visible) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    *total = 0;
    if (visible) *visible = 0;
  }
}

struct SortedCountLoad {
  const int* counts;
  const int* order;
  __device__ int64_t operator()(int64_t j) const { return counts[order[j]]; }
};

// starts[j] = entries of all lower depth ranks (pair_keys_kernel has
// already summed the total M).
struct ExclusiveStartStore {
  int64_t* starts;
  __device__ void operator()(int64_t j, int64_t inclusive, int64_t v) const {
    starts[j] = inclusive - v;
  }
};

// Stage 2, step 1: lane j of the grid takes depth rank j (its pair, the
// rectangle stage 1 stored and its first entry) and writes the pair's tiles
// row-major as 32-bit tile ids plus the pair index. A pair with at most
// `lane_tiles` tiles is written by its own lane; larger ones are written by
// the whole wave, one pair at a time, 64 consecutive entries per store, so
// that a few huge rectangles do not serialise their wave. Entries at or
// past m (inconsistent inputs) are dropped. The limit only distributes the
// work: every entry is written to the same place whatever it is.
// kLaneTiles suits rectangles of ~18 tiles on average (1M surfels at
// 1080p); scenes whose mean rectangle exceeds kWideMean tiles emit faster
// with kWideLaneTiles (the host picks it when it knows M and V).
constexpr int kLaneTiles = 32;
constexpr int kWideLaneTiles = 8;
constexpr int kWideMean = 24;

// `m` is the capacity of tile_ids/values; `total` (a device int64, or null
// when it equals m) the emission's full length, which may exceed it: entries
// past the capacity are dropped and `status` (if given) gets kBinOverflow.
// A depth-sort output outside [0, count) is replaced by pair 0 and sets
// kBinBadIndex (index_guard.hpp).
// Packed: instead of (tile id, pair index) pairs, write one 32-bit key
// tile id << rank_bits | depth rank per entry (the caller has checked that
// both fit), so that the tile sort moves keys only; values is unused.
template <bool Packed>
__global__ __launch_bounds__(256) void emit_sorted_kernel(
    int64_t count, int64_t m, const int64_t* __restrict__ total_count, uint32_t* status,
    int tw, const int* __restrict__ order, const int64_t* __restrict__ starts,
    const int4* __restrict__ rects, uint32_t* __restrict__ tile_ids, int* __restrict__ values,
    int rank_bits, int lane_tiles) {
  const int lane = __lane_id();
  const int64_t j = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (j - lane >= count) return;  // uniform per wave
  const int64_t total = total_count ? *total_count : m;
  if (status && j == 0 && total > m) atomicOr(status, kBinOverflow);
  int pair = 0, area = 0;
  int4 rect = make_int4(0, 0, 1, 0);
  int64_t first = 0;
  if (j < count) {
    bool bad = false;
    pair = checked_index(order[j], count, bad);
    if (bad && status) atomicOr(status, kBinBadIndex);
    first = starts[j];
    const int64_t next = j + 1 < count ? starts[j + 1] : total;
    area = int(min<int64_t>(next - first, INT_MAX));
    if (area > 0) rect = rects[pair];
  }
  // Packed entries carry the depth rank j in their low bits.
  const uint32_t low = uint32_t(j);
  if (area <= lane_tiles) {
    int x = rect.x, y = rect.y;
    for (int k = 0; k < area; ++k) {
      const int64_t e = first + k;
      if (e < m) {
        const uint32_t tile = uint32_t(rect.w) + uint32_t(y * tw + x);
        if constexpr (Packed) {
          tile_ids[e] = (tile << rank_bits) | low;
        } else {
          tile_ids[e] = tile;
          values[e] = pair;
        }
      }
      if (++x == rect.x + rect.z) {
        x = rect.x;
        ++y;
      }
    }
  }
  uint64_t big = __ballot(area > lane_tiles);
  while (big) {  // uniform: every lane sees the same mask
    const int owner = __ffsll((unsigned long long)big) - 1;
    big &= big - 1;
    const int64_t owner_first = __shfl(first, owner);
    const int owner_area = __shfl(area, owner);
    const int owner_x0 = __shfl(rect.x, owner);
    const int owner_y0 = __shfl(rect.y, owner);
    const int owner_span = __shfl(rect.z, owner);
    const uint32_t owner_base = uint32_t(__shfl(rect.w, owner));
    const int owner_pair = __shfl(pair, owner);
    const uint32_t owner_low = uint32_t(__shfl(int(low), owner));
    for (int k = lane; k < owner_area; k += 64) {
      const int64_t e = owner_first + k;
      if (e < m) {
        const uint32_t tile = owner_base + uint32_t((owner_y0 + k / owner_span) * tw + owner_x0 +
                                                    k % owner_span);
        if constexpr (Packed) {
          tile_ids[e] = (tile << rank_bits) | owner_low;
        } else {
          tile_ids[e] = tile;
          values[e] = owner_pair;
        }
      }
    }
  }
}

// Tile ranges from the tile-sorted entries. Packed: the entries are
// tile id << rank_bits | depth rank keys, and this pass also writes the
// point list, point_list[i] = order[rank]. Either way every point-list
// entry is checked against the pair count `count` before the compositors
// dereference it: a depth rank or pair index outside [0, count) is replaced
// by 0 and sets kBinBadIndex in `status` (if given).
template <bool Packed>
__global__ __launch_bounds__(256) void find_tile_ranges_kernel(int64_t capacity,
                                                               const int64_t* __restrict__ live,
                                                               int64_t tiles,
                                                               const uint32_t* __restrict__ ids,
                                                               int2* __restrict__ ranges,
                                                               int rank_bits,
                                                               const int* __restrict__ order,
                                                               int* __restrict__ point_list,
                                                               int64_t count,
                                                               uint32_t* status) {
  const int64_t m = live ? min(capacity, max(*live, int64_t(0))) : capacity;
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= m) {
    // Bounded binning: the entries past the live count are defined as -1.
    if (i < capacity) point_list[i] = -1;
    return;
  }
  const uint32_t key = ids[i];
  const uint32_t tile = Packed ? key >> rank_bits : key;
  bool bad = false;
  if constexpr (Packed) {
    const int rank = checked_index(packed_rank(key, rank_bits), count, bad);
    point_list[i] = checked_index(order[rank], count, bad);
  } else {
    const int pair = point_list[i];
    const int safe = checked_index(pair, count, bad);
    if (bad) point_list[i] = safe;
  }
  if (bad && status) atomicOr(status, kBinBadIndex);
  const bool own = tile < uint64_t(tiles);
  if (i == 0) {
    if (own) ranges[tile].x = 0;
  } else {
    const uint32_t previous = Packed ? ids[i - 1] >> rank_bits : ids[i - 1];
    if (tile != previous) {
      if (previous < uint64_t(tiles)) ranges[previous].y = int(i);
      if (own) ranges[tile].x = int(i);
    }
  }
  if (i == m - 1 && own) ranges[tile].y = int(m);
}

struct OrderWorkspace {
  uint32_t* keys;      // count
  uint32_t* sorted;    // count
  int* pair_ids;       // count
  int* counts;         // count
  int64_t* scan_sums;
  void* sort;          // radix sort scratch for count keys
  long long* partials;  // [ceil(count / 256)][2]: pair_keys_kernel's workgroup totals
  size_t bytes;
};

OrderWorkspace order_layout(void* base, int64_t count) {
  OrderWorkspace w;
  char* p = static_cast<char*>(base);
  size_t offset = 0;
  auto take = [&](size_t bytes) {
    char* at = p + offset;
    offset = align_up(offset + bytes, 256);
    return at;
  };
  w.keys = reinterpret_cast<uint32_t*>(take(size_t(count) * 4));
  w.sorted = reinterpret_cast<uint32_t*>(take(size_t(count) * 4));
  w.pair_ids = reinterpret_cast<int*>(take(size_t(count) * 4));
  w.counts = reinterpret_cast<int*>(take(size_t(count) * 4));
  w.scan_sums = reinterpret_cast<int64_t*>(take(scan_workspace_bytes(count, 8)));
  w.sort = take(radix_sort_workspace_bytes(count, 4));
  w.partials = reinterpret_cast<long long*>(take(size_t(ceil_div(count, 256)) * 16));
  w.bytes = offset;
  return w;
}

struct TilesWorkspace {
  uint32_t* tile_ids;     // m, depth order
  int* tile_values;       // m
  uint32_t* tile_sorted;  // m, tile order
  void* sort;             // radix sort scratch for m keys
  size_t bytes;
};

TilesWorkspace tiles_layout(void* base, int64_t m) {
  TilesWorkspace w;
  char* p = static_cast<char*>(base);
  size_t offset = 0;
  auto take = [&](size_t bytes) {
    char* at = p + offset;
    offset = align_up(offset + bytes, 256);
    return at;
  };
  w.tile_ids = reinterpret_cast<uint32_t*>(take(size_t(m) * 4));
  w.tile_values = reinterpret_cast<int*>(take(size_t(m) * 4));
  w.tile_sorted = reinterpret_cast<uint32_t*>(take(size_t(m) * 4));
  w.sort = take(radix_sort_workspace_bytes(m, 4));
  w.bytes = offset;
  return w;
}

// Bits needed for ids below `tiles`.
int id_bits(int64_t tiles) {
  int bits = 0;
  while (bits < 63 && (int64_t(1) << bits) < tiles) ++bits;
  return bits;
}

}  // namespace
}  // namespace gs

extern "C" {

size_t gs_scan_workspace_size(int64_t count) {
  return gs::scan_workspace_bytes(count, sizeof(int64_t));
}

int gs_pack_visible(const int32_t* radii, int64_t count, int64_t* selected,
                    int32_t* row_of_pair, int64_t* num_selected, void* workspace,
                    size_t workspace_bytes, void* stream) {
  using namespace gs;
  clear_error();
  GS_REQUIRE(count >= 0 && count <= INT_MAX, GS_ERR_OVERFLOW, "too many pairs to pack");
  GS_REQUIRE(num_selected, GS_ERR_ARGUMENT, "null num_selected");
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_BINNING, s);
  if (count == 0) {
    zero_count_kernel<<<1, 64, 0, s>>>(num_selected);
    GS_LAUNCHED("zero_count_kernel");
    return GS_OK;
  }
  GS_REQUIRE(radii && selected, GS_ERR_ARGUMENT, "null pointer passed to gs_pack_visible");
  const size_t need = gs_scan_workspace_size(count);
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE,
             "packing needs %zu workspace bytes, got %zu", need, workspace_bytes);
  return run_scan<int64_t>(count, VisibleLoad{radii},
                           SelectStore{selected, row_of_pair, num_selected, count},
                           static_cast<int64_t*>(workspace), s);
}

int gs_count_tiles(const float* geometry, const int32_t* radii, int64_t count, int32_t width,
                   int32_t height, int64_t* offsets, void* workspace, size_t workspace_bytes,
                   void* stream) {
  using namespace gs;
  clear_error();
  GS_REQUIRE(count >= 0 && count <= INT_MAX, GS_ERR_OVERFLOW, "too many projected primitives");
  GS_REQUIRE(width > 0 && height > 0, GS_ERR_ARGUMENT, "invalid image dimensions");
  if (count == 0) return GS_OK;
  GS_REQUIRE(geometry && radii && offsets, GS_ERR_ARGUMENT,
             "null pointer passed to gs_count_tiles");
  const size_t need = gs_scan_workspace_size(count);
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE,
             "tile count needs %zu workspace bytes, got %zu", need, workspace_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_BINNING, s);
  return run_scan<int64_t>(count, TileCountLoad{geometry, radii, tiles_x(width), tiles_y(height)},
                           InclusiveStore{offsets}, static_cast<int64_t*>(workspace), s);
}

int gs_emit_tiles(const float* geometry, const int32_t* radii, const int64_t* image_ids,
                  const int64_t* offsets, int64_t count, int32_t width, int32_t height,
                  uint64_t* keys, int32_t* values, void* stream) {
  using namespace gs;
  clear_error();
  GS_REQUIRE(count >= 0 && count <= INT_MAX, GS_ERR_OVERFLOW, "too many projected primitives");
  GS_REQUIRE(width > 0 && height > 0, GS_ERR_ARGUMENT, "invalid image dimensions");
  if (count == 0) return GS_OK;
  GS_REQUIRE(geometry && radii && image_ids && offsets && keys && values, GS_ERR_ARGUMENT,
             "null pointer passed to gs_emit_tiles");
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_BINNING, s);
  emit_tiles_kernel<<<unsigned(ceil_div(count, 256)), 256, 0, s>>>(
      count, tiles_x(width), tiles_y(height), geometry, radii, image_ids, offsets, keys, values);
  GS_LAUNCHED("emit_tiles_kernel");
  return GS_OK;
}

int gs_find_ranges(const uint64_t* sorted_keys, int64_t m, int32_t* ranges, int64_t tiles,
                   void* stream) {
  using namespace gs;
  clear_error();
  GS_REQUIRE(m >= 0 && m <= INT_MAX, GS_ERR_OVERFLOW, "tile intersection count exceeds int32");
  GS_REQUIRE(tiles >= 0 && tiles <= INT_MAX, GS_ERR_OVERFLOW, "image tile count exceeds int32");
  if (tiles == 0) return GS_OK;
  GS_REQUIRE(ranges, GS_ERR_ARGUMENT, "null ranges");
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_BINNING, s);
  int2* r = reinterpret_cast<int2*>(ranges);
  fill_ranges_kernel<<<unsigned(ceil_div(tiles, 256)), 256, 0, s>>>(tiles, r);
  GS_LAUNCHED("fill_ranges_kernel");
  if (m == 0) return GS_OK;
  GS_REQUIRE(sorted_keys, GS_ERR_ARGUMENT, "null sorted keys");
  find_ranges_kernel<<<unsigned(ceil_div(m, 256)), 256, 0, s>>>(m, tiles, sorted_keys, r);
  GS_LAUNCHED("find_ranges_kernel");
  return GS_OK;
}

size_t gs_bin_order_workspace_size(int64_t count) {
  if (count < 0) count = 0;
  return gs::order_layout(nullptr, count).bytes + 256;
}

int gs_bin_order_count(const float* geometry, const int32_t* radii, const int64_t* image_ids,
                       int64_t count, int32_t width, int32_t height, int32_t* rects,
                       int64_t* intersections, int64_t* visible, void* workspace,
                       size_t workspace_bytes, void* stream) {
  using namespace gs;
  clear_error();
  GS_REQUIRE(count >= 0 && count <= INT_MAX, GS_ERR_OVERFLOW, "too many projected primitives");
  GS_REQUIRE(width > 0 && height > 0, GS_ERR_ARGUMENT, "invalid image dimensions");
  GS_REQUIRE(intersections, GS_ERR_ARGUMENT, "null intersections");
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_BINNING, s);
  if (count == 0) {
    zero_totals_kernel<<<1, 64, 0, s>>>(intersections, visible);
    GS_LAUNCHED("zero_totals_kernel");
    return GS_OK;
  }
  GS_REQUIRE(geometry && radii && image_ids && rects, GS_ERR_ARGUMENT,
             "null pointer passed to gs_bin_order_count");
  const size_t need = gs_bin_order_workspace_size(count);
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE,
             "binning needs %zu workspace bytes, got %zu", need, workspace_bytes);
  OrderWorkspace w = order_layout(workspace, count);
  const int64_t blocks = ceil_div(count, 256);
  pair_keys_kernel<<<unsigned(blocks), 256, 0, s>>>(
      count, tiles_x(width), tiles_y(height), geometry, radii, image_ids, w.keys, w.pair_ids,
      w.counts, reinterpret_cast<int4*>(rects), w.partials);
  GS_LAUNCHED("pair_keys_kernel");
  totals_kernel<<<1, kTotalsBlock, 0, s>>>(w.partials, blocks, intersections, visible);
  GS_LAUNCHED("totals_kernel");
  return GS_OK;
}

int gs_bin_order_sort(int64_t count, int32_t* order, int64_t* starts, void* workspace,
                      size_t workspace_bytes, void* stream) {
  using namespace gs;
  clear_error();
  GS_REQUIRE(count >= 0 && count <= INT_MAX, GS_ERR_OVERFLOW, "too many projected primitives");
  if (count == 0) return GS_OK;
  GS_REQUIRE(order && starts, GS_ERR_ARGUMENT, "null pointer passed to gs_bin_order_sort");
  const size_t need = gs_bin_order_workspace_size(count);
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE,
             "binning needs %zu workspace bytes, got %zu", need, workspace_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  OrderWorkspace w = order_layout(workspace, count);
  {
    ProfileScope prof(GS_PROF_SORT, s);
    int status = radix_sort<uint32_t>(w.keys, w.sorted, w.pair_ids, order, count, 0, 32, w.sort,
                                      s);
    if (status != GS_OK) return status;
  }
  ProfileScope prof(GS_PROF_BINNING, s);
  return run_scan<int64_t>(count, SortedCountLoad{w.counts, order}, ExclusiveStartStore{starts},
                           w.scan_sums, s);
}

int gs_bin_order(const float* geometry, const int32_t* radii, const int64_t* image_ids,
                 int64_t count, int32_t width, int32_t height, int32_t* order, int64_t* starts,
                 int32_t* rects, int64_t* intersections, int64_t* visible, void* workspace,
                 size_t workspace_bytes, void* stream) {
  using namespace gs;
  clear_error();
  GS_REQUIRE(count >= 0 && count <= INT_MAX, GS_ERR_OVERFLOW, "too many projected primitives");
  GS_REQUIRE(count == 0 || (order && starts), GS_ERR_ARGUMENT,
             "null pointer passed to gs_bin_order");
  const int status = gs_bin_order_count(geometry, radii, image_ids, count, width, height, rects,
                                        intersections, visible, workspace, workspace_bytes,
                                        stream);
  if (status != GS_OK) return status;
  return gs_bin_order_sort(count, order, starts, workspace, workspace_bytes, stream);
}

size_t gs_bin_tiles_workspace_size(int64_t m) {
  if (m < 0) m = 0;
  return gs::tiles_layout(nullptr, m).bytes + 256;
}

}  // extern "C"

namespace gs {
namespace {

// Shared by gs_bin_tiles (m known on the host) and gs_bin_tiles_bounded (m
// a capacity, the live length in `live` on the device).
// `visible`: the number of pairs with tiles (stage 1's V), or -1 when only
// the device knows it. Pairs with tiles hold depth ranks below V (below
// count when V is unknown); when those ranks and the tile ids fit in 32 bits
// together, the entries travel as packed keys (emit_sorted_kernel<true>).
int bin_tiles(const int32_t* order, const int64_t* starts, const int32_t* rects, int64_t count,
              int64_t m, const int64_t* live, uint32_t* status, int64_t images, int32_t width,
              int32_t height, int32_t* point_list, int32_t* ranges, int64_t visible,
              void* workspace, size_t workspace_bytes, hipStream_t s) {
  GS_REQUIRE(count >= 0 && count <= INT_MAX, GS_ERR_OVERFLOW, "too many projected primitives");
  GS_REQUIRE(m >= 0 && m <= INT_MAX, GS_ERR_OVERFLOW, "tile intersection count exceeds int32");
  GS_REQUIRE(width > 0 && height > 0 && images >= 0, GS_ERR_ARGUMENT,
             "invalid image dimensions");
  const int tw = tiles_x(width), th = tiles_y(height);
  const int64_t tiles = images * int64_t(tw) * int64_t(th);
  GS_REQUIRE(tiles <= INT_MAX, GS_ERR_OVERFLOW, "image tile count exceeds int32");
  if (status) {
    clear_flag_kernel<<<1, 64, 0, s>>>(status);
    GS_LAUNCHED("clear_flag_kernel");
  }
  if (tiles == 0) return GS_OK;
  GS_REQUIRE(ranges, GS_ERR_ARGUMENT, "null ranges");
  const size_t need = gs_bin_tiles_workspace_size(m);
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE,
             "binning needs %zu workspace bytes, got %zu", need, workspace_bytes);
  int2* r = reinterpret_cast<int2*>(ranges);
  TilesWorkspace w = tiles_layout(workspace, m);
  const int tile_bits = id_bits(tiles);
  const int rank_bits = id_bits(visible >= 0 ? min(visible, count) : count);
  const bool packed = tile_bits + rank_bits <= 32;
  const int lane_tiles =
      (!live && visible > 0 && m > int64_t(kWideMean) * visible) ? kWideLaneTiles : kLaneTiles;
  const int4* rect_rows = reinterpret_cast<const int4*>(rects);
  {
    ProfileScope prof(GS_PROF_BINNING, s);
    fill_ranges_kernel<<<unsigned(ceil_div(tiles, 256)), 256, 0, s>>>(tiles, r);
    GS_LAUNCHED("fill_ranges_kernel");
    if (count == 0 || (m == 0 && !live)) return GS_OK;
    GS_REQUIRE(order && starts && rects, GS_ERR_ARGUMENT, "null pointer passed to gs_bin_tiles");
    if (m == 0) {  // a zero capacity still reports an overflowing emission
      emit_sorted_kernel<false><<<unsigned(ceil_div(count, 256)), 256, 0, s>>>(
          count, 0, live, status, tw, order, starts, rect_rows, nullptr, nullptr, 0, lane_tiles);
      GS_LAUNCHED("emit_sorted_kernel");
      return GS_OK;
    }
    GS_REQUIRE(point_list, GS_ERR_ARGUMENT, "null point list");
    if (packed) {
      emit_sorted_kernel<true><<<unsigned(ceil_div(count, 256)), 256, 0, s>>>(
          count, m, live, status, tw, order, starts, rect_rows, w.tile_ids, nullptr,
          rank_bits, lane_tiles);
    } else {
      emit_sorted_kernel<false><<<unsigned(ceil_div(count, 256)), 256, 0, s>>>(
          count, m, live, status, tw, order, starts, rect_rows, w.tile_ids, w.tile_values, 0,
          lane_tiles);
    }
    GS_LAUNCHED("emit_sorted_kernel");
  }
  {
    ProfileScope prof(GS_PROF_SORT, s);
    // Stable on the tile bits: entries of a tile keep their depth order.
    const int sorted =
        packed ? radix_sort<uint32_t>(w.tile_ids, w.tile_sorted, nullptr, nullptr, m, rank_bits,
                                      rank_bits + tile_bits, w.sort, s, live)
               : radix_sort<uint32_t>(w.tile_ids, w.tile_sorted, w.tile_values, point_list, m, 0,
                                      tile_bits, w.sort, s, live);
    if (sorted != GS_OK) return sorted;
  }
  ProfileScope prof(GS_PROF_BINNING, s);
  if (packed) {
    find_tile_ranges_kernel<true><<<unsigned(ceil_div(m, 256)), 256, 0, s>>>(
        m, live, tiles, w.tile_sorted, r, rank_bits, order, point_list, count, status);
  } else {
    find_tile_ranges_kernel<false><<<unsigned(ceil_div(m, 256)), 256, 0, s>>>(
        m, live, tiles, w.tile_sorted, r, 0, nullptr, point_list, count, status);
  }
  GS_LAUNCHED("find_tile_ranges_kernel");
  return GS_OK;
}

}  // namespace
}  // namespace gs

extern "C" {

int gs_bin_tiles(const int32_t* order, const int64_t* starts, const int32_t* rects,
                 int64_t count, int64_t m, int64_t visible, int64_t images, int32_t width,
                 int32_t height, int32_t* point_list, int32_t* ranges, uint32_t* status,
                 void* workspace, size_t workspace_bytes, void* stream) {
  gs::clear_error();
  return gs::bin_tiles(order, starts, rects, count, m, nullptr, status, images, width, height,
                       point_list, ranges, visible, workspace, workspace_bytes,
                       static_cast<hipStream_t>(stream));
}

int gs_bin_tiles_bounded(const int32_t* order, const int64_t* starts, const int32_t* rects,
                         int64_t count, int64_t capacity, const int64_t* intersections,
                         int64_t images, int32_t width, int32_t height, int32_t* point_list,
                         int32_t* ranges, uint32_t* overflow, void* workspace,
                         size_t workspace_bytes, void* stream) {
  gs::clear_error();
  GS_REQUIRE(intersections && overflow, GS_ERR_ARGUMENT,
             "bounded binning needs the device intersection count and an overflow flag");
  return gs::bin_tiles(order, starts, rects, count, capacity, intersections, overflow, images,
                       width, height, point_list, ranges, -1, workspace, workspace_bytes,
                       static_cast<hipStream_t>(stream));
}

}  // extern "C"
