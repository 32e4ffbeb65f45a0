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
// Three binning pipelines give the same point list and ranges:
//  * reference order (gs_emit_tiles, gs_sort_pairs, gs_find_ranges): every
//    pair emits one 64-bit (image|tile) << 32 | depth-bits key per covered
//    tile, and the M keys are radix-sorted on 32 + bits(tiles) bits;
//  * depth first, tile path (gs_bin_order, then gs_bin_tiles): the Q pairs
//    are stably sorted on their depth bits, each pair then emits its tiles
//    in that order as 32-bit tile ids, and a stable sort on only
//    bits(tiles) bits groups them by tile. The first stage needs no
//    intersection count; M and V are summed by its first kernels, so the
//    host reads them while the depth sort runs. A stable sort of
//    depth-ordered entries by tile leaves each tile's entries ordered by
//    (depth bits, pair index) - the order of the 64-bit sort - while the M
//    entries move through two 8-bit passes of 8 bytes instead of 5-6
//    passes of 12 bytes;
//  * depth first, block path (gs_bin_blocks_*), the renderer's wherever
//    the image has at most 65,536 tile blocks: the same depth order, then
//    one entry per 4 x 4-tile block a pair meets (about M / 6 of them),
//    sorted by block, and each block's entries written into its tiles'
//    lists (see the block path's stage 2 below). Its bounded form
//    (gs_bin_blocks_tiles_bounded), like gs_bin_tiles_bounded, reads the
//    counts on the device, for callers that cannot synchronise.
#include <climits>
#include <cmath>
#include <cstring>

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

// Bounded binning with nothing to bin (no pairs, or a zero capacity): the
// point list's `capacity` entries past the live count are -1, and a live
// count above the capacity sets kBinOverflow. The grid covers
// max(capacity, 1) threads.
__global__ __launch_bounds__(256) void bounded_tail_kernel(int* __restrict__ list,
                                                           int64_t capacity,
                                                           const int64_t* __restrict__ live,
                                                           uint32_t* status) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t m = *live;
  if (i == 0 && m > capacity && status) atomicOr(status, kBinOverflow);
  if (i < capacity && i >= max(m, int64_t(0))) list[i] = -1;
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

// Tile blocks: kBlockSide x kBlockSide tiles of one image, numbered row-major
// per image and image after image. The block path bins the pairs into
// blocks first and then each block's pairs into its tiles.
constexpr int kBlockShift = 2;
constexpr int kBlockSide = 1 << kBlockShift;
__host__ __device__ inline int blocks_across(int tiles) { return (tiles + kBlockSide - 1) >> kBlockShift; }

// Blocks met by the tile rectangle [x0, x1) x [y0, y1) (non-empty, in one
// image's tile coordinates).
__device__ __forceinline__ int block_area(int x0, int y0, int x1, int y1) {
  return (((x1 - 1) >> kBlockShift) - (x0 >> kBlockShift) + 1) *
         (((y1 - 1) >> kBlockShift) - (y0 >> kBlockShift) + 1);
}

// Depth-first binning, stage 1, step 1: each pair's tile rectangle, its
// entry count and its depth key; pairs without tiles sort last.
//  * tile path (Blocks = false): rects[i] = (x0, y0, width, first tile id of
//    its image) and counts[i] = the rectangle's area (countTiles);
//  * block path (Blocks = true): rects[i] = (x0, y0 + image*th, x1, y1 +
//    image*th), the rectangle in the images' tile rows stacked top to
//    bottom, and counts[i] = the number of tile blocks it meets.
// Each workgroup also stores its sums of the tile counts, of the pairs with
// tiles and of the block counts in partials[block], which totals_kernel adds
// up into M, V and the block entries, so the host can read them before the
// pairs are sorted (plain stores and one more launch: thousands of
// workgroups adding into one device word would queue their atomics behind
// each other).
// Block path depth keys: float bits of the depth minus `depth_base`, the
// depth clamped to [depth_base, depth_limit] first (see DepthKeys).
template <bool Blocks>
__global__ __launch_bounds__(256) void pair_keys_kernel(int64_t count, int tw, int th,
                                                        const float* __restrict__ geometry,
                                                        const int* __restrict__ radii,
                                                        const int64_t* __restrict__ image_ids,
                                                        uint32_t* __restrict__ keys,
                                                        int* __restrict__ values,
                                                        int* __restrict__ counts,
                                                        int4* __restrict__ rects,
                                                        long long* __restrict__ partials,
                                                        uint32_t depth_base,
                                                        uint32_t depth_limit) {
  __shared__ long long wave_sums[3][4];
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  int c = 0, b = 0;
  if (i < count) {
    const int r = radii[i];
    uint32_t key = 0xffffffffu;
    int4 rect = Blocks ? make_int4(0, 0, 0, 0) : make_int4(0, 0, 1, 0);
    if (r > 0) {
      const float* g = geometry + i * kGeometry;
      const TileRect t = tile_rect(g[9], g[10], r, tw, th);
      c = (t.x1 - t.x0) * (t.y1 - t.y0);
      if (c > 0) {
        key = __float_as_uint(g[8]);
        if constexpr (Blocks) {
          key = min(max(key, depth_base), depth_limit) - depth_base;
          b = block_area(t.x0, t.y0, t.x1, t.y1);
          const int rows = int(image_ids[i]) * th;
          rect = make_int4(t.x0, t.y0 + rows, t.x1, t.y1 + rows);
        } else {
          rect = make_int4(t.x0, t.y0, t.x1 - t.x0, int(image_ids[i] * int64_t(tw) * th));
        }
      }
    }
    counts[i] = Blocks ? b : c;
    keys[i] = key;
    values[i] = int(i);
    rects[i] = rect;
  }
  // Workgroup totals: wave sums by shuffles, then across the four waves.
  long long sum = c, with_tiles = c > 0 ? 1 : 0, block_sum = b;
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    sum += __shfl_xor(sum, offset, 64);
    with_tiles += __shfl_xor(with_tiles, offset, 64);
    block_sum += __shfl_xor(block_sum, offset, 64);
  }
  const int wave = threadIdx.x >> 6;
  if (__lane_id() == 0) {
    wave_sums[0][wave] = sum;
    wave_sums[1][wave] = with_tiles;
    wave_sums[2][wave] = block_sum;
  }
  __syncthreads();
  if (threadIdx.x < 3)
    partials[3 * int64_t(blockIdx.x) + threadIdx.x] =
        wave_sums[threadIdx.x][0] + wave_sums[threadIdx.x][1] + wave_sums[threadIdx.x][2] +
        wave_sums[threadIdx.x][3];
}

// M, V and the block entries from pair_keys_kernel's `blocks` workgroup
// totals (one workgroup; `visible` and `block_total` may be null).
constexpr int kTotalsBlock = 1024;
__global__ __launch_bounds__(kTotalsBlock) void totals_kernel(const long long* __restrict__ partials,
                                                             int64_t blocks, int64_t* total,
                                                             int64_t* visible,
                                                             int64_t* block_total) {
  __shared__ long long wave_sums[3][kTotalsBlock / 64];
  long long sums[3] = {0, 0, 0};
  for (int64_t b = threadIdx.x; b < blocks; b += kTotalsBlock) {
#pragma unroll
    for (int k = 0; k < 3; ++k) sums[k] += partials[3 * b + k];
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) sums[k] += __shfl_xor(sums[k], offset, 64);
    if (__lane_id() == 0) wave_sums[k][threadIdx.x >> 6] = sums[k];
  }
  __syncthreads();
  if (threadIdx.x < 3) {
    long long value = 0;
#pragma unroll
    for (int w = 0; w < kTotalsBlock / 64; ++w) value += wave_sums[threadIdx.x][w];
    int64_t* target = threadIdx.x == 0 ? total : threadIdx.x == 1 ? visible : block_total;
    if (target) *target = value;
  }
}

// No pairs: M = V = 0 (and no block entries).
__global__ __launch_bounds__(64) void zero_totals_kernel(int64_t* total, int64_t* visible,
                                                         int64_t* block_total) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    *total = 0;
    if (visible) *visible = 0;
    if (block_total) *block_total = 0;
  }
}

// counts[order[j]]; an order entry outside [0, count) counts 0 here (the
// emission flags it).
struct SortedCountLoad {
  const int* counts;
  const int* order;
  int64_t count;
  __device__ int64_t operator()(int64_t j) const {
    const int pair = order[j];
    return pair >= 0 && pair < count ? counts[pair] : 0;
  }
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

// --------------------------------------------------------------------------
// Block path, stage 2. Stage 1 (pair_keys_kernel<true>, the depth sort and
// the scan of block counts) leaves the pairs in depth order with the first
// block entry of each. Then:
//  1. emit_blocks_kernel writes, rank after rank, one entry per tile block a
//     pair's rectangle meets: key = block id << 16 | the 16-bit mask of the
//     block's tiles the rectangle covers (bit 4 ly + lx), value = pair;
//  2. a stable sort on the block-id bits groups the entries by block, each
//     block's entries staying in depth order;
//  3. block_bounds_kernel finds where each block's entries start;
//  4. block_tile_count_kernel counts each tile's entries per chunk of its
//     block's list (one wave per chunk, each for all 16 tiles of the block),
//     and a scan of the tile totals gives the tile ranges;
//  5. block_tile_write_kernel: the same waves walk their chunks again and
//     write the pairs whose mask covers each tile, in list order, from the
//     tile's range start plus its entries in the earlier chunks.
// Every tile's list is then its pairs in (depth bits, pair index) order, as
// with the tile sort, while the sort moves about M / 6 entries instead of M
// (a pair meets ~18 tiles but ~3 blocks on a 1080p scene of 1M surfels).

// Mask of the tiles of block (bx, by) that [x0, x1) x [y0, y1) covers.
__device__ __forceinline__ uint32_t block_mask(int bx, int by, int x0, int y0, int x1, int y1) {
  const int lx0 = max(x0 - (bx << kBlockShift), 0), lx1 = min(x1 - (bx << kBlockShift), kBlockSide);
  const int ly0 = max(y0 - (by << kBlockShift), 0), ly1 = min(y1 - (by << kBlockShift), kBlockSide);
  const uint32_t columns = ((1u << lx1) - 1u) & ~((1u << lx0) - 1u);
  const uint32_t rows = ((1u << (kBlockSide * ly1)) - 1u) & ~((1u << (kBlockSide * ly0)) - 1u);
  return (columns * 0x1111u) & rows;
}

// One lane per depth rank below `ranks` (the pairs with tiles) reads its
// pair and rectangle; the wave then writes its 64 ranks' entries, which are
// consecutive in the output, together, 64 consecutive entries per store:
// lane i of a round takes entry wave_first + 64 r + i, finds the rank that
// owns it (a binary search over the lanes' first entries by shuffles) and
// that rank's rectangle (shuffles). Entries at or past `capacity` are
// dropped. A depth-sort output outside [0, count) is replaced by pair 0 and
// sets kBinBadIndex; its scanned block count was 0, so it writes nothing.
// The entry total is `total`, or *live_total (a device word) when that is
// given; a live total above `capacity` sets kBinOverflow.
constexpr int kMaskBits = 16;

__global__ __launch_bounds__(256) void emit_blocks_kernel(
    int64_t ranks, int64_t count, int64_t capacity, int64_t total,
    const int64_t* __restrict__ live_total, uint32_t* status, int th, int bw, int bh,
    const int* __restrict__ order, const int64_t* __restrict__ starts,
    const int4* __restrict__ rects, uint32_t* __restrict__ keys, int* __restrict__ values) {
  const int lane = __lane_id();
  const int64_t j = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t wave_rank = j - lane;
  if (wave_rank >= ranks) return;  // uniform per wave
  if (live_total) {
    total = *live_total;
    if (j == 0 && total > capacity && status) atomicOr(status, kBinOverflow);
  }
  const int last = int(min<int64_t>(63, ranks - 1 - wave_rank));  // last lane with a rank
  int pair = 0, area = 0, bx0 = 0, by0 = 0, span = 1, x0 = 0, y0 = 0, x1 = 0, y1 = 0;
  uint32_t base = 0;
  int64_t first = 0;
  if (lane <= last) {
    bool bad = false;
    pair = checked_index(order[j], count, bad);
    if (bad && status) atomicOr(status, kBinBadIndex);
    first = starts[j];
    const int64_t next = j + 1 < count ? starts[j + 1] : total;
    area = int(max<int64_t>(min<int64_t>(next - first, INT_MAX), 0));
    if (area > 0) {
      const int4 r = rects[pair];
      const int image = r.y / th;
      x0 = r.x;
      x1 = r.z;
      y0 = r.y - image * th;
      y1 = r.w - image * th;
      bx0 = x0 >> kBlockShift;
      by0 = y0 >> kBlockShift;
      span = ((x1 - 1) >> kBlockShift) - bx0 + 1;
      base = uint32_t(image) * uint32_t(bw) * uint32_t(bh);
    }
  }
  const int64_t wave_first = __shfl(first, 0);
  const int64_t wave_end = __shfl(first + area, last);
  // Offsets from the wave's first entry (the wave's entries number below
  // 2^31: they are part of at most `capacity` <= INT_MAX).
  const int offset = int(first - wave_first);
  for (int64_t e = wave_first + lane; e - lane < wave_end; e += 64) {
    const int want = int(e - wave_first);
    int owner = 0;  // last lane whose first entry is at or before e
#pragma unroll
    for (int step = 32; step > 0; step >>= 1) {
      const int probe = owner + step;
      const int at = __shfl(offset, probe <= last ? probe : last);
      if (probe <= last && at <= want) owner = probe;
    }
    const int k = want - __shfl(offset, owner);
    const int o_bx0 = __shfl(bx0, owner), o_by0 = __shfl(by0, owner);
    const int o_span = __shfl(span, owner);
    const int ox0 = __shfl(x0, owner), oy0 = __shfl(y0, owner);
    const int ox1 = __shfl(x1, owner), oy1 = __shfl(y1, owner);
    const uint32_t o_base = uint32_t(__shfl(int(base), owner));
    const int o_pair = __shfl(pair, owner);
    if (e < wave_end && e >= 0 && e < capacity) {
      const int bx = o_bx0 + k % o_span, by = o_by0 + k / o_span;
      keys[e] = ((o_base + uint32_t(by * bw + bx)) << kMaskBits) |
                block_mask(bx, by, ox0, oy0, ox1, oy1);
      values[e] = o_pair;
    }
  }
}

// min(capacity, *live) clamped at 0, or capacity without a live word.
__device__ __forceinline__ int64_t live_entries(int64_t capacity, const int64_t* live) {
  return live ? min(capacity, max(*live, int64_t(0))) : capacity;
}

// first[b] = index of block b's first entry in the block-sorted keys, for
// b in [0, blocks]; empty blocks start where the next entry is (first[blocks]
// = m, m = the entry count: live_entries(capacity, live)). Each entry whose
// block differs from its predecessor's writes the starts of the blocks from
// just after the predecessor's to its own. The same launch clears
// tile_counts (`tiles` entries) for block_tile_count_kernel's atomic sums
// and, for bounded binning (tail non-null), sets the point-list entries
// [live_entries(tail_capacity, tail_live), tail_capacity) to -1. Every
// thread strides over the grid, which may be smaller than the work (bounded
// binning caps it: its capacities are sizes, not counts).
__global__ __launch_bounds__(256) void block_bounds_kernel(
    int64_t capacity, const int64_t* __restrict__ live, int64_t blocks,
    const uint32_t* __restrict__ keys, int* __restrict__ first, int64_t tiles,
    int* __restrict__ tile_counts, int* __restrict__ tail, int64_t tail_capacity,
    const int64_t* __restrict__ tail_live) {
  const int64_t stride = int64_t(gridDim.x) * 256;
  const int64_t gid = int64_t(blockIdx.x) * 256 + threadIdx.x;
  for (int64_t i = gid; i < tiles; i += stride) tile_counts[i] = 0;
  if (tail)
    for (int64_t i = live_entries(tail_capacity, tail_live) + gid; i < tail_capacity; i += stride)
      tail[i] = -1;
  const int64_t m = live_entries(capacity, live);
  if (m == 0) {  // no entries (bounded binning): every block is empty
    for (int64_t b = gid; b <= blocks; b += stride) first[b] = 0;
    return;
  }
  for (int64_t i = gid; i < m; i += stride) {
    const int64_t block = min<int64_t>(keys[i] >> kMaskBits, blocks);
    const int64_t previous = i == 0 ? -1 : min<int64_t>(keys[i - 1] >> kMaskBits, blocks);
    for (int64_t b = previous + 1; b <= block; ++b) first[b] = int(i);
    if (i == m - 1)
      for (int64_t b = block + 1; b <= blocks; ++b) first[b] = int(m);
  }
}

// Workgroups of block_bounds_kernel in bounded binning (8 per CU).
constexpr int64_t kBoundedBoundsGroups = 2048;

// The tiles of block b: local tile k = 4 ly + lx (its bit in an entry's
// mask) is tile (4 bx + lx, 4 by + ly) of the block's image.
constexpr int kBlockTiles = kBlockSide * kBlockSide;

struct BlockTiles {
  int image, tx, ty;  // image, first tile of the block
  __device__ BlockTiles(int64_t block, int bw, int bh) {
    const int64_t per_image = int64_t(bw) * bh;
    image = int(block / per_image);
    const int rest = int(block - image * per_image);
    tx = (rest % bw) << kBlockShift;
    ty = (rest / bw) << kBlockShift;
  }
  __device__ bool inside(int k, int tw, int th) const {
    return tx + (k & (kBlockSide - 1)) < tw && ty + (k >> kBlockShift) < th;
  }
  __device__ int64_t tile(int k, int tw, int th) const {
    return (int64_t(image) * th + ty + (k >> kBlockShift)) * tw + tx + (k & (kBlockSide - 1));
  }
};

// The block's entry list is cut into kChunks contiguous chunks of
// max(kChunkMin, ceil(length / kChunks)) entries (the last ones shorter or
// empty); workgroup g of a block
// has kChunkWaves waves, and wave w takes chunk kChunkWaves g + w (empty
// when the list has fewer chunks) for all 16 tiles of the block, 64 entries
// per step and up to kWaveSteps steps per round, all of a round's loads
// issued before any is used. No wave waits for another.
constexpr int kChunks = 16;
constexpr int kChunkMin = 256;
constexpr int kChunkWaves = 4;
constexpr int kChunkGroups = kChunks / kChunkWaves;
constexpr int kWaveSteps = 16;

struct BlockChunk {
  int64_t block;
  int chunk, begin, end;  // chunk of the block list, its entries [begin, end)
  __device__ BlockChunk(const int* first) {
    block = blockIdx.x / kChunkGroups;
    chunk = int(blockIdx.x % kChunkGroups) * kChunkWaves + (int(threadIdx.x) >> 6);
    const int list_begin = first[block], list_end = first[block + 1];
    const int length = list_end - list_begin;
    // ceil(length / kChunks), but at least kChunkMin: later chunks may be
    // shorter or empty.
    const int64_t chunk_length = max<int64_t>(kChunkMin, (int64_t(length) + kChunks - 1) / kChunks);
    begin = list_begin + int(min<int64_t>(length, chunk * chunk_length));
    end = list_begin + int(min<int64_t>(length, (chunk + 1) * chunk_length));
  }
};

// chunk_counts[(b kChunks + c) 16 + k] = entries of chunk c of block b whose
// mask has local tile k's bit; tile_counts[t] (cleared by
// block_bounds_kernel) += the same, summed over the chunks by atomics.
__global__ __launch_bounds__(kChunkWaves * 64) void block_tile_count_kernel(
    int bw, int bh, int tw, int th, const int* __restrict__ first,
    const uint32_t* __restrict__ keys, int* __restrict__ chunk_counts,
    int* __restrict__ tile_counts) {
  const BlockChunk part(first);
  const int lane = __lane_id();
  int c[kBlockTiles] = {};
  for (int base = part.begin; base < part.end; base += 64 * kWaveSteps) {
    uint32_t key[kWaveSteps];
#pragma unroll
    for (int u = 0; u < kWaveSteps; ++u) {
      const int i = base + u * 64 + lane;
      key[u] = i < part.end ? keys[i] : 0u;
    }
    const int steps = (part.end - base + 63) >> 6;  // uniform
#pragma unroll
    for (int u = 0; u < kWaveSteps; ++u) {
      if (u >= steps) break;
#pragma unroll
      for (int k = 0; k < kBlockTiles; ++k) c[k] += int((key[u] >> k) & 1u);
    }
  }
  int mine = 0;  // lane k < 16: local tile k's count
#pragma unroll
  for (int k = 0; k < kBlockTiles; ++k) {
    int v = c[k];
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    mine = lane == k ? v : mine;
  }
  if (lane < kBlockTiles) {
    chunk_counts[(part.block * kChunks + part.chunk) * kBlockTiles + lane] = mine;
    const BlockTiles tiles(part.block, bw, bh);
    if (mine > 0 && tiles.inside(lane, tw, th))
      atomicAdd(&tile_counts[tiles.tile(lane, tw, th)], mine);
  }
}

struct TileTotalLoad {
  const int* counts;
  __device__ int64_t operator()(int64_t t) const { return counts[t]; }
};

// ranges[t] = [first, last) of tile t's entries, (0, 0) for an empty tile;
// clamped to the point list's m entries (only a point list shorter than
// the entries, as bounded binning's capacity can be, reaches the clamp), so
// that no range leaves the list and every slot a range covers is written.
// A tile with entries keeps its clamped start even when nothing of it is
// left (m, m): block_tile_write_kernel starts the tile's slots there, so
// they all fall at or past m and are dropped, not written over the front of
// the list.
struct TileRangeStore {
  int2* ranges;
  int64_t m;
  __device__ void operator()(int64_t t, int64_t inclusive, int64_t v) const {
    const int64_t first = min(inclusive - v, m), last = min(inclusive, m);
    ranges[t] = v > 0 ? make_int2(int(first), int(last)) : make_int2(0, 0);
  }
};

// Tile ranges of up to kRangeItems * 1024 tiles in one workgroup and one
// pass: thread t takes tiles [kRangeItems t, kRangeItems (t + 1)), adds its
// counts, and a workgroup scan of those sums gives each thread its first
// entry; ranges as TileRangeStore writes them.
constexpr int kRangeThreads = 1024;
constexpr int kRangeItems = 8;
constexpr int64_t kRangeLocalTiles = int64_t(kRangeThreads) * kRangeItems;

__global__ __launch_bounds__(kRangeThreads) void tile_ranges_local_kernel(
    int64_t tiles, int64_t m, const int* __restrict__ counts, int2* __restrict__ ranges) {
  __shared__ int64_t wave_totals[kRangeThreads / 64];
  const int lane = __lane_id(), wave = threadIdx.x >> 6;
  const int64_t t0 = int64_t(threadIdx.x) * kRangeItems;
  int c[kRangeItems];
  int64_t sum = 0;
#pragma unroll
  for (int u = 0; u < kRangeItems; ++u) {
    c[u] = t0 + u < tiles ? counts[t0 + u] : 0;
    sum += c[u];
  }
  const int64_t inclusive = wave_inclusive_scan(sum);
  if (lane == 63) wave_totals[wave] = inclusive;
  __syncthreads();
  int64_t at = inclusive - sum;
  for (int w = 0; w < wave; ++w) at += wave_totals[w];
  const TileRangeStore store{ranges, m};
#pragma unroll
  for (int u = 0; u < kRangeItems; ++u) {
    at += c[u];
    if (t0 + u < tiles) store(t0 + u, at, c[u]);
  }
}

// Each wave writes its chunk's part of the block's 16 tile lists: the pairs
// of the entries whose mask has a tile's bit, in block-list order, from the
// tile's range start plus the tile's entries in the block's earlier chunks
// (ballot + lane prefix per step and tile). Positions at or past m are
// dropped and set kBinOverflow; a pair outside [0, count) is replaced by
// pair 0 and sets kBinBadIndex.
__global__ __launch_bounds__(kChunkWaves * 64) void block_tile_write_kernel(
    int bw, int bh, int tw, int th, const int* __restrict__ first,
    const uint32_t* __restrict__ keys, const int* __restrict__ values,
    const int2* __restrict__ ranges, const int* __restrict__ chunk_counts,
    int* __restrict__ point_list, int m, int count, uint32_t* status) {
  const BlockChunk part(first);
  if (part.begin >= part.end) return;  // uniform per wave; no barrier here
  const BlockTiles tiles(part.block, bw, bh);
  const int lane = __lane_id();
  // Lane k < 16: local tile k's first slot for this chunk. Unsigned: a slot
  // that wraps on inconsistent inputs is >= m and dropped.
  uint32_t start = 0;
  const bool inside = lane < kBlockTiles && tiles.inside(lane, tw, th);
  if (inside) {
    start = uint32_t(ranges[tiles.tile(lane, tw, th)].x);
    // The earlier chunks' counts: all loads issued at once.
    const int* column = chunk_counts + part.block * kChunks * kBlockTiles + lane;
#pragma unroll
    for (int c = 0; c < kChunks - 1; ++c)
      start += c < part.chunk ? uint32_t(column[c * kBlockTiles]) : 0u;
  }
  const uint32_t inside_bits = uint32_t(__ballot(inside));
  uint32_t next[kBlockTiles];
#pragma unroll
  for (int k = 0; k < kBlockTiles; ++k) next[k] = uint32_t(__shfl(int(start), k));
  bool bad = false, overflow = false;
  for (int base = part.begin; base < part.end; base += 64 * kWaveSteps) {
    uint32_t key[kWaveSteps];
    int pair[kWaveSteps];
#pragma unroll
    for (int u = 0; u < kWaveSteps; ++u) {
      const int i = base + u * 64 + lane;
      key[u] = i < part.end ? keys[i] : 0u;
      pair[u] = checked_index(i < part.end ? values[i] : 0, count, bad);
    }
    const int steps = (part.end - base + 63) >> 6;  // uniform
#pragma unroll
    for (int u = 0; u < kWaveSteps; ++u) {
      if (u >= steps) break;
      const uint32_t mask = key[u] & inside_bits;
#pragma unroll
      for (int k = 0; k < kBlockTiles; ++k) {
        const bool take = (mask >> k) & 1u;
        const uint64_t vote = __ballot(take);
        const uint32_t slot = __builtin_amdgcn_mbcnt_hi(
            uint32_t(vote >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(vote), next[k]));
        if (take && slot < uint32_t(m)) point_list[slot] = pair[u];
        next[k] += uint32_t(__popcll(vote));
      }
    }
  }
  // A tile whose slots ran past m dropped entries (uniform: next[k] is the
  // same in every lane, and it never wraps: starts <= m, m + entries < 2^32).
#pragma unroll
  for (int k = 0; k < kBlockTiles; ++k) overflow |= next[k] > uint32_t(m);
  if (status && (bad || overflow))
    atomicOr(status, (bad ? kBinBadIndex : 0u) | (overflow ? kBinOverflow : 0u));
}

struct OrderWorkspace {
  uint32_t* keys;      // count
  uint32_t* sorted;    // count
  int* pair_ids;       // count
  int* counts;         // count
  int64_t* scan_sums;
  void* sort;          // radix sort scratch for count keys
  long long* partials;  // [ceil(count / 256)][3]: pair_keys_kernel's workgroup totals
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
  w.partials = reinterpret_cast<long long*>(take(size_t(ceil_div(count, 256)) * 24));
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

struct BlocksWorkspace {
  uint32_t* keys;         // block entries, depth order
  int* values;
  uint32_t* sorted_keys;  // block order
  int* sorted_values;
  void* sort;             // radix sort scratch
  int* first;             // blocks + 1
  int* chunk_counts;      // blocks * kChunks * 16
  int* tile_counts;       // tiles
  int64_t* scan_sums;     // tile-count scan
  size_t bytes;
};

BlocksWorkspace blocks_layout(void* base, int64_t entries, int64_t blocks, int64_t tiles) {
  BlocksWorkspace w;
  char* p = static_cast<char*>(base);
  size_t offset = 0;
  auto take = [&](size_t bytes) {
    char* at = p + offset;
    offset = align_up(offset + bytes, 256);
    return at;
  };
  w.keys = reinterpret_cast<uint32_t*>(take(size_t(entries) * 4));
  w.values = reinterpret_cast<int*>(take(size_t(entries) * 4));
  w.sorted_keys = reinterpret_cast<uint32_t*>(take(size_t(entries) * 4));
  w.sorted_values = reinterpret_cast<int*>(take(size_t(entries) * 4));
  w.sort = take(radix_sort_workspace_bytes(entries, 4));
  w.first = reinterpret_cast<int*>(take(size_t(blocks + 1) * 4));
  w.chunk_counts = reinterpret_cast<int*>(take(size_t(blocks) * kChunks * kBlockTiles * 4));
  w.tile_counts = reinterpret_cast<int*>(take(size_t(tiles) * 4));
  w.scan_sums = reinterpret_cast<int64_t*>(take(scan_workspace_bytes(tiles, 8)));
  w.bytes = offset;
  return w;
}

// Tile blocks of `images` images of tw x th tiles.
int64_t block_count(int64_t images, int tw, int th) {
  return images * int64_t(blocks_across(tw)) * int64_t(blocks_across(th));
}

// Bits needed for ids below `tiles`.
int id_bits(int64_t tiles) {
  int bits = 0;
  while (bits < 63 && (int64_t(1) << bits) < tiles) ++bits;
  return bits;
}

// Depth keys of the block path. Pairs with tiles are visible, so their
// depth z lies in (near, far); for near > 0 the float bits of those depths
// form the contiguous range (bits(near), bits(far)), and bits(z) -
// bits(near) orders them as the raw bits do in fewer bits: bits(far) -
// bits(near) + 1 values, 27 bits for the default planes (0.2, 100), so the
// depth sort takes three 9-bit passes instead of four 8-bit ones. Pairs
// without tiles keep key 0xffffffff, whose low `bits` bits exceed every
// visible key. Otherwise (near <= 0 or planes not finite) the raw bits on
// all 32 bits.
struct DepthKeys {
  uint32_t base = 0, limit = 0xffffffffu;
  int bits = 32;
  DepthKeys(float near_plane, float far_plane) {
    if (!(near_plane > 0.f) || !(far_plane > near_plane) || !std::isfinite(far_plane)) return;
    uint32_t lo, hi;
    std::memcpy(&lo, &near_plane, 4);
    std::memcpy(&hi, &far_plane, 4);
    const uint64_t span = uint64_t(hi - lo) + 1;  // key values 0..hi-lo, then the sentinel
    int b = 0;
    while (b < 32 && (uint64_t(1) << b) <= span) ++b;
    if (b >= 32) return;
    base = lo;
    limit = hi;
    bits = b;
  }
};

// Stage 1's first step for both paths (pair_keys_kernel<Blocks>, then the
// totals; every total pointer but `intersections` may be null).
template <bool Blocks>
int order_count(const float* geometry, const int32_t* radii, const int64_t* image_ids,
                int64_t count, int32_t width, int32_t height, int32_t* rects,
                int64_t* intersections, int64_t* visible, int64_t* block_total, void* workspace,
                size_t workspace_bytes, hipStream_t s, DepthKeys depth = DepthKeys(0.f, 0.f)) {
  GS_REQUIRE(count >= 0 && count <= INT_MAX, GS_ERR_OVERFLOW, "too many projected primitives");
  GS_REQUIRE(width > 0 && height > 0, GS_ERR_ARGUMENT, "invalid image dimensions");
  GS_REQUIRE(intersections, GS_ERR_ARGUMENT, "null intersections");
  ProfileScope prof(GS_PROF_BINNING, s);
  if (count == 0) {
    zero_totals_kernel<<<1, 64, 0, s>>>(intersections, visible, block_total);
    GS_LAUNCHED("zero_totals_kernel");
    return GS_OK;
  }
  GS_REQUIRE(geometry && radii && image_ids && rects, GS_ERR_ARGUMENT,
             "null pointer passed to gs_bin_order_count");
  const size_t need = order_layout(nullptr, count).bytes + 256;
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE,
             "binning needs %zu workspace bytes, got %zu", need, workspace_bytes);
  OrderWorkspace w = order_layout(workspace, count);
  const int64_t blocks = ceil_div(count, 256);
  pair_keys_kernel<Blocks><<<unsigned(blocks), 256, 0, s>>>(
      count, tiles_x(width), tiles_y(height), geometry, radii, image_ids, w.keys, w.pair_ids,
      w.counts, reinterpret_cast<int4*>(rects), w.partials, depth.base, depth.limit);
  GS_LAUNCHED("pair_keys_kernel");
  totals_kernel<<<1, kTotalsBlock, 0, s>>>(w.partials, blocks, intersections, visible,
                                           block_total);
  GS_LAUNCHED("totals_kernel");
  return GS_OK;
}

// Stage 1's second step: the depth order of the pairs (keys on bits
// [0, key_bits)) and the exclusive scan of their counts in that order.
int order_sort(int64_t count, int key_bits, int32_t* order, int64_t* starts, void* workspace,
               size_t workspace_bytes, hipStream_t s) {
  GS_REQUIRE(count >= 0 && count <= INT_MAX, GS_ERR_OVERFLOW, "too many projected primitives");
  if (count == 0) return GS_OK;
  GS_REQUIRE(order && starts, GS_ERR_ARGUMENT, "null pointer passed to gs_bin_order_sort");
  const size_t need = order_layout(nullptr, count).bytes + 256;
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE,
             "binning needs %zu workspace bytes, got %zu", need, workspace_bytes);
  OrderWorkspace w = order_layout(workspace, count);
  {
    ProfileScope prof(GS_PROF_SORT, s);
    int status = radix_sort<uint32_t>(w.keys, w.sorted, w.pair_ids, order, count, 0, key_bits,
                                      w.sort, s);
    if (status != GS_OK) return status;
  }
  ProfileScope prof(GS_PROF_BINNING, s);
  return run_scan<int64_t>(count, SortedCountLoad{w.counts, order, count},
                           ExclusiveStartStore{starts}, w.scan_sums, s);
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
  gs::clear_error();
  return gs::order_count<false>(geometry, radii, image_ids, count, width, height, rects,
                                intersections, visible, nullptr, workspace, workspace_bytes,
                                static_cast<hipStream_t>(stream));
}

int gs_bin_blocks_fit(int64_t images, int32_t width, int32_t height) {
  if (images < 0 || width <= 0 || height <= 0) return 0;
  return gs::block_count(images, gs::tiles_x(width), gs::tiles_y(height)) <=
                 (int64_t(1) << (32 - gs::kMaskBits))
             ? 1
             : 0;
}

int gs_bin_blocks_count(const float* geometry, const int32_t* radii, const int64_t* image_ids,
                        int64_t count, int32_t width, int32_t height, float near_plane,
                        float far_plane, int32_t* rects, int64_t* totals, void* workspace,
                        size_t workspace_bytes, void* stream) {
  using namespace gs;
  clear_error();
  GS_REQUIRE(totals, GS_ERR_ARGUMENT, "null totals");
  return order_count<true>(geometry, radii, image_ids, count, width, height, rects, totals,
                           totals + 1, totals + 2, workspace, workspace_bytes,
                           static_cast<hipStream_t>(stream), DepthKeys(near_plane, far_plane));
}

int gs_bin_order_sort(int64_t count, int32_t* order, int64_t* starts, void* workspace,
                      size_t workspace_bytes, void* stream) {
  gs::clear_error();
  return gs::order_sort(count, 32, order, starts, workspace, workspace_bytes,
                        static_cast<hipStream_t>(stream));
}

int gs_bin_blocks_sort(int64_t count, float near_plane, float far_plane, int32_t* order,
                       int64_t* starts, void* workspace, size_t workspace_bytes, void* stream) {
  gs::clear_error();
  return gs::order_sort(count, gs::DepthKeys(near_plane, far_plane).bits, order, starts,
                        workspace, workspace_bytes, static_cast<hipStream_t>(stream));
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
    if (count == 0 && live && m > 0) {  // nothing binned: the whole list is -1
      GS_REQUIRE(point_list, GS_ERR_ARGUMENT, "null point list");
      bounded_tail_kernel<<<unsigned(ceil_div(m, 256)), 256, 0, s>>>(point_list, m, live,
                                                                     status);
      GS_LAUNCHED("bounded_tail_kernel");
    }
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

namespace gs {
namespace {

// Shared by gs_bin_blocks_tiles (m and entries known on the host) and
// gs_bin_blocks_tiles_bounded (totals: the device words M, V, E of
// gs_bin_blocks_count; m is the point list's capacity, and the block entries
// are sized for as many, since E <= M).
int bin_blocks_tiles(const int32_t* order, const int64_t* starts, const int32_t* rects,
                     int64_t count, int64_t m, int64_t entries, int64_t visible, int64_t images,
                     int32_t width, int32_t height, int32_t* point_list, int32_t* ranges,
                     uint32_t* status, void* workspace, size_t workspace_bytes, hipStream_t s,
                     const int64_t* totals = nullptr) {
  GS_REQUIRE(count >= 0 && count <= INT_MAX, GS_ERR_OVERFLOW, "too many projected primitives");
  GS_REQUIRE(m >= 0 && m <= INT_MAX, GS_ERR_OVERFLOW, "tile intersection count exceeds int32");
  GS_REQUIRE(entries >= 0 && entries <= INT_MAX, GS_ERR_OVERFLOW,
             "tile block entry count exceeds int32");
  GS_REQUIRE(width > 0 && height > 0 && images >= 0, GS_ERR_ARGUMENT,
             "invalid image dimensions");
  const int tw = tiles_x(width), th = tiles_y(height);
  const int64_t tiles = images * int64_t(tw) * int64_t(th);
  GS_REQUIRE(tiles <= INT_MAX, GS_ERR_OVERFLOW, "image tile count exceeds int32");
  const int bw = blocks_across(tw), bh = blocks_across(th);
  const int64_t blocks = block_count(images, tw, th);
  GS_REQUIRE(blocks <= (int64_t(1) << (32 - kMaskBits)), GS_ERR_ARGUMENT,
             "%lld tile blocks exceed the block path's %lld", (long long)blocks,
             (long long)(int64_t(1) << (32 - kMaskBits)));
  if (status) {
    clear_flag_kernel<<<1, 64, 0, s>>>(status);
    GS_LAUNCHED("clear_flag_kernel");
  }
  if (tiles == 0) return GS_OK;
  GS_REQUIRE(ranges, GS_ERR_ARGUMENT, "null ranges");
  const size_t need = blocks_layout(nullptr, entries, blocks, tiles).bytes + 256;
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE,
             "binning needs %zu workspace bytes, got %zu", need, workspace_bytes);
  int2* r = reinterpret_cast<int2*>(ranges);
  BlocksWorkspace w = blocks_layout(workspace, entries, blocks, tiles);
  // Bounded: the live entry count E (capped at `entries`) and M.
  const int64_t* live_e = totals ? totals + 2 : nullptr;
  const int64_t* live_m = totals;
  if (count == 0 || entries == 0) {
    ProfileScope prof(GS_PROF_BINNING, s);
    fill_ranges_kernel<<<unsigned(ceil_div(tiles, 256)), 256, 0, s>>>(tiles, r);
    GS_LAUNCHED("fill_ranges_kernel");
    if (totals) {  // a -1 list, and an overflow when M exceeds a zero capacity
      GS_REQUIRE(m == 0 || point_list, GS_ERR_ARGUMENT, "null point list");
      bounded_tail_kernel<<<unsigned(ceil_div(max(m, int64_t(1)), 256)), 256, 0, s>>>(
          point_list, m, live_m, status);
      GS_LAUNCHED("bounded_tail_kernel");
    }
    return GS_OK;
  }
  GS_REQUIRE(order && starts && rects && point_list, GS_ERR_ARGUMENT,
             "null pointer passed to gs_bin_blocks_tiles");
  const int64_t ranks = visible >= 0 ? min(visible, count) : count;
  {
    ProfileScope prof(GS_PROF_BINNING, s);
    if (ranks > 0) {
      emit_blocks_kernel<<<unsigned(ceil_div(ranks, 256)), 256, 0, s>>>(
          ranks, count, entries, entries, live_e, status, th, bw, bh, order, starts,
          reinterpret_cast<const int4*>(rects), w.keys, w.values);
      GS_LAUNCHED("emit_blocks_kernel");
    }
  }
  {
    ProfileScope prof(GS_PROF_SORT, s);
    // Stable on the block bits: entries of a block keep their depth order.
    const int sorted = radix_sort<uint32_t>(w.keys, w.sorted_keys, w.values, w.sorted_values,
                                            entries, kMaskBits, kMaskBits + id_bits(blocks),
                                            w.sort, s, live_e);
    if (sorted != GS_OK) return sorted;
  }
  ProfileScope prof(GS_PROF_BINNING, s);
  const int64_t bound_threads = max(max(entries, tiles), max(blocks + 1, totals ? m : 0));
  const int64_t bound_groups = ceil_div(bound_threads, 256);
  block_bounds_kernel<<<unsigned(totals ? min(bound_groups, kBoundedBoundsGroups)
                                        : bound_groups),
                        256, 0, s>>>(
      entries, live_e, blocks, w.sorted_keys, w.first, tiles, w.tile_counts,
      totals ? point_list : nullptr, m, live_m);
  GS_LAUNCHED("block_bounds_kernel");
  const unsigned groups = unsigned(blocks * kChunkGroups);
  block_tile_count_kernel<<<groups, kChunkWaves * 64, 0, s>>>(
      bw, bh, tw, th, w.first, w.sorted_keys, w.chunk_counts, w.tile_counts);
  GS_LAUNCHED("block_tile_count_kernel");
  if (tiles <= kRangeLocalTiles) {
    tile_ranges_local_kernel<<<1, kRangeThreads, 0, s>>>(tiles, m, w.tile_counts, r);
    GS_LAUNCHED("tile_ranges_local_kernel");
  } else {
    const int scanned = run_scan<int64_t>(tiles, TileTotalLoad{w.tile_counts},
                                          TileRangeStore{r, m}, w.scan_sums, s);
    if (scanned != GS_OK) return scanned;
  }
  block_tile_write_kernel<<<groups, kChunkWaves * 64, 0, s>>>(
      bw, bh, tw, th, w.first, w.sorted_keys, w.sorted_values, r, w.chunk_counts, point_list,
      int(m), int(count), status);
  GS_LAUNCHED("block_tile_write_kernel");
  return GS_OK;
}

}  // namespace
}  // namespace gs

extern "C" {

size_t gs_bin_blocks_tiles_workspace_size(int64_t entries, int64_t images, int32_t width,
                                          int32_t height) {
  if (entries < 0) entries = 0;
  if (images < 0 || width <= 0 || height <= 0) return 256;
  const int tw = gs::tiles_x(width), th = gs::tiles_y(height);
  return gs::blocks_layout(nullptr, entries, gs::block_count(images, tw, th),
                           images * int64_t(tw) * th)
             .bytes +
         256;
}

int gs_bin_blocks_tiles(const int32_t* order, const int64_t* starts, const int32_t* rects,
                        int64_t count, int64_t m, int64_t entries, int64_t visible,
                        int64_t images, int32_t width, int32_t height, int32_t* point_list,
                        int32_t* ranges, uint32_t* status, void* workspace,
                        size_t workspace_bytes, void* stream) {
  gs::clear_error();
  return gs::bin_blocks_tiles(order, starts, rects, count, m, entries, visible, images, width,
                              height, point_list, ranges, status, workspace, workspace_bytes,
                              static_cast<hipStream_t>(stream));
}

int gs_bin_blocks_tiles_bounded(const int32_t* order, const int64_t* starts,
                                const int32_t* rects, int64_t count, int64_t capacity,
                                const int64_t* totals, int64_t images, int32_t width,
                                int32_t height, int32_t* point_list, int32_t* ranges,
                                uint32_t* overflow, void* workspace, size_t workspace_bytes,
                                void* stream) {
  gs::clear_error();
  GS_REQUIRE(totals && overflow, GS_ERR_ARGUMENT,
             "bounded binning needs the device totals and an overflow flag");
  return gs::bin_blocks_tiles(order, starts, rects, count, capacity, capacity, -1, images,
                              width, height, point_list, ranges, overflow, workspace,
                              workspace_bytes, static_cast<hipStream_t>(stream), totals);
}

}  // extern "C"
