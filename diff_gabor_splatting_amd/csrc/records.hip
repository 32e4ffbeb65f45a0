// Kernel 1 (fused): projection + SH + record assembly, and its adjoint.
//
// Replaces the reference's host-side chain (src/gabor_splatting/rendering.py:
// 323-374): project_surfaces, SHColors, the per-camera expansion of the
// shared appearance and opacity, the packing gathers and the geometry
// concatenation. One thread per (scene, surfel) loops over the cameras of
// its scene and writes each pair's compositor rows directly:
//   geometry [Q,17] = T | xy | facing normal | unit direction,
//   projected means [Q,2], radii [Q], image ids [Q], primitive ids [Q],
//   and with SH: appearance rows [Q,18] = colour(3) colour2(3) weights(4)
//   magnitudes(4) phases(4) and opacity rows [Q] (camera-specific colours).
// Rows are dense (row = pair index (s*C + c)*N + n) or, in packed mode,
// compacted through row_of_pair (visible pairs only, in ascending pair
// order, exactly the reference's `arange(Q)[radii > 0]`). Packed SH rows are
// compacted too (the reference keeps them dense), and each row's
// primitive id is then the row itself. A dense row whose pair is culled
// (radius 0) is referenced by no tile list: it gets its radius, projected
// mean and ids, zero geometry and appearance rows (written with its
// neighbours' in whole cache lines) and no opacity entry.
//
// The adjoint reads the compositor's gradient rows: an SH pass sums colour
// and shared-parameter gradients over cameras per surfel (no atomics) and
// leaves per-pair direction gradients in the workspace; the projection
// adjoint (projection.hpp) then consumes transform / normal / direction rows
// and the projected-mean gradients.
#include "projection.hpp"
#include "sh_basis.hpp"

namespace gs {
namespace {

constexpr int kRow = kClassic;  // SH appearance row width

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// One thread per (scene, surfel) loops over the cameras of its scene. Every
// pair gets its radius, projected mean and ids; pairs that reach a tile
// (radius > 0) also get their geometry row and, with SH, their appearance
// and opacity rows. The SH coefficients of culled pairs are never read. Coefficients are read one colour
// set at a time, in 16-byte vectors when the set's length allows.
template <int KC, bool Vec>
__device__ __forceinline__ void load_coefficients(const float* __restrict__ src, float* dst) {
  if constexpr (Vec && KC % 4 == 0) {
    const float4* v = reinterpret_cast<const float4*>(src);
#pragma unroll
    for (int i = 0; i < KC / 4; ++i) {
      const float4 q = v[i];
      dst[4 * i + 0] = q.x;
      dst[4 * i + 1] = q.y;
      dst[4 * i + 2] = q.z;
      dst[4 * i + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < KC; ++i) dst[i] = src[i];
  }
}

// Vec: the SH coefficient and shared-parameter arrays start on 16-byte
// boundaries, so that 16-byte vector loads are legal.
// Row staging: each thread leaves its pair's geometry row (17 floats) and,
// with SH, appearance row (18) in LDS at an odd pitch, and the workgroup
// then writes the rows of its 256 consecutive pairs with consecutive
// threads on consecutive floats - the rows of consecutive pairs are
// consecutive in both dense and packed mode - skipping culled pairs.
template <int Width>
__device__ __forceinline__ void unstage_pair_rows(const float* stage, int pitch, int offset,
                                                  const int64_t* rows, float* __restrict__ out) {
#pragma unroll 4
  for (int e = threadIdx.x; e < kProjectBlock * Width; e += kProjectBlock) {
    const int local = e / Width, f = e - local * Width;
    const int64_t row = rows[local];
    if (row >= 0) out[row * Width + f] = stage[local * pitch + offset + f];
  }
}

// Dense rows (row == pair): a workgroup's rows [first, first + count) are
// one contiguous run, written whole with 16-byte stores (rows of culled
// pairs as zeros), so that every store fills whole cache lines.
template <int Width>
__device__ __forceinline__ void unstage_dense_rows(const float* stage, int pitch, int offset,
                                                   const int64_t* rows, int64_t first, int count,
                                                   float* __restrict__ out) {
  float* dst = out + first * Width;
  const int total = count * Width;
  auto value = [&](int e) {
    const int local = e / Width, f = e - local * Width;
    return rows[local] >= 0 ? stage[local * pitch + offset + f] : 0.f;
  };
  const int head = min(int((4u - ((reinterpret_cast<uintptr_t>(dst) >> 2) & 3u)) & 3u), total);
  if (int(threadIdx.x) < head) dst[threadIdx.x] = value(threadIdx.x);
  const int body = (total - head) / 4;
  float4* dst4 = reinterpret_cast<float4*>(dst + head);
  for (int q = threadIdx.x; q < body; q += kProjectBlock) {
    const int e = head + 4 * q;
    dst4[q] = make_float4(value(e), value(e + 1), value(e + 2), value(e + 3));
  }
  const int tail = head + 4 * body;
  if (tail + int(threadIdx.x) < total) dst[tail + threadIdx.x] = value(tail + threadIdx.x);
}

template <int Degree, bool Vec>  // Degree -1: no SH rows
__global__ __launch_bounds__(kProjectBlock) void records_forward_kernel(
    const float* __restrict__ means, const float* __restrict__ quats,
    const float* __restrict__ scales, const float* __restrict__ opacities,
    const float* __restrict__ views, const float* __restrict__ intrinsics,
    const float* __restrict__ sh_first, const float* __restrict__ sh_second,
    const float* __restrict__ weights, const float* __restrict__ magnitudes,
    const float* __restrict__ phases, int64_t cameras, int64_t n, int tw, int th,
    float near_plane, float far_plane, const int* __restrict__ row_of_pair,
    int* __restrict__ dense_radii, float* __restrict__ geometry,
    float* __restrict__ projected_means, int* __restrict__ row_radii,
    int64_t* __restrict__ primitive_ids, int64_t* __restrict__ image_ids,
    float* __restrict__ appearance, float* __restrict__ opacity_rows,
    int64_t* __restrict__ meta_scene_ids, int64_t* __restrict__ meta_camera_ids,
    int64_t* __restrict__ meta_surfel_ids) {
  constexpr bool kSH = Degree >= 0;
  constexpr int K = kSH ? (Degree + 1) * (Degree + 1) : 1;
  constexpr int KC = K * 3;
  constexpr int kPitch = kSH ? kGeometry + kRow : kGeometry;  // 35 or 17: odd
  __shared__ float stage[kProjectBlock * kPitch];
  __shared__ int64_t stage_rows[kProjectBlock];
  const int t = threadIdx.x;
  const int64_t i = int64_t(blockIdx.x) * kProjectBlock + t;
  const int64_t scene = blockIdx.y;
  const bool own = i < n;
  const int64_t surfel = scene * n + i;
  Surfel s;
  if (own) load_surfel(means, quats, scales, surfel, s);
  for (int64_t c = 0; c < cameras; ++c) {  // uniform: every thread takes part in the staging
    const int64_t cam = scene * cameras + c;
    int64_t staged = -1;
    if (own) {
      Projection p;
      project_pair(s.R, s.mu, s.sc, views + cam * 16, intrinsics + cam * 9, p);
      const int64_t pair = cam * n + i;
      const int radius = screen_radius(p, tw, th, near_plane, far_plane);
      if (dense_radii) dense_radii[pair] = radius;
      const int64_t row = !geometry ? -1 : row_of_pair ? int64_t(row_of_pair[pair]) : pair;
      if (row >= 0) {
        projected_means[row * 2 + 0] = p.xy[0];
        projected_means[row * 2 + 1] = p.xy[1];
        row_radii[row] = radius;
        image_ids[row] = cam;
        primitive_ids[row] = kSH ? row : surfel;
        if (meta_scene_ids) {
          meta_scene_ids[row] = scene;
          meta_camera_ids[row] = c;
          meta_surfel_ids[row] = i;
        }
      }
      if (row >= 0 && radius > 0) {
        staged = row;
        float* g = stage + t * kPitch;
#pragma unroll
        for (int k = 0; k < 9; ++k) g[k] = p.T[k];
        g[9] = p.xy[0];
        g[10] = p.xy[1];
        const float sign = facing_sign(p);
#pragma unroll
        for (int k = 0; k < 3; ++k) g[11 + k] = p.nraw[k] * sign;
        float d[3];
        unit_direction(p, d);
#pragma unroll
        for (int k = 0; k < 3; ++k) g[14 + k] = d[k];
        if constexpr (kSH) {
          float Y[K];
          sh_basis<(kSH ? Degree : 0), false>(d[0], d[1], d[2], Y, nullptr, nullptr, nullptr);
          float* a = g + kGeometry;
#pragma unroll
          for (int set = 0; set < 2; ++set) {
            float coef[KC];
            load_coefficients<KC, Vec>((set ? sh_second : sh_first) + surfel * KC, coef);
#pragma unroll
            for (int ch = 0; ch < 3; ++ch) {
              float raw = 0.5f;
#pragma unroll
              for (int k = 0; k < K; ++k) raw += Y[k] * coef[k * 3 + ch];
              a[set * 3 + ch] = fmaxf(raw, 0.f);
            }
          }
          float shared[12];
          load_coefficients<4, Vec>(weights + surfel * 4, shared);
          load_coefficients<4, Vec>(magnitudes + surfel * 4, shared + 4);
          load_coefficients<4, Vec>(phases + surfel * 4, shared + 8);
#pragma unroll
          for (int k = 0; k < 12; ++k) a[6 + k] = shared[k];
          opacity_rows[row] = opacities[surfel];
        }
      }
    }
    if (!geometry) continue;  // uniform: a radii-only pass writes no rows
    stage_rows[t] = staged;
    __syncthreads();
    if (!row_of_pair) {
      const int64_t first = cam * n + int64_t(blockIdx.x) * kProjectBlock;
      const int count = int(min<int64_t>(kProjectBlock, n - int64_t(blockIdx.x) * kProjectBlock));
      unstage_dense_rows<kGeometry>(stage, kPitch, 0, stage_rows, first, count, geometry);
      if constexpr (kSH)
        unstage_dense_rows<kRow>(stage, kPitch, kGeometry, stage_rows, first, count, appearance);
    } else {
      unstage_pair_rows<kGeometry>(stage, kPitch, 0, stage_rows, geometry);
      if constexpr (kSH) unstage_pair_rows<kRow>(stage, kPitch, kGeometry, stage_rows, appearance);
    }
    __syncthreads();  // the next camera overwrites the stage
  }
}

// SH part of the adjoint: per surfel, sum over cameras the colour gradients
// pushed through the basis (coefficients), the shared weight / magnitude /
// phase and opacity gradients; write per-pair direction gradients.
//
// One workgroup handles 64 consecutive surfels. Each colour set's
// coefficients (3K floats per surfel, contiguous across the block) are read
// with coalesced loads into LDS, rows of odd pitch so that every lane then
// reads its own surfel without bank conflicts, and the coefficient
// gradients leave the same way.
// Surfels whose colour gradients are all zero in every camera (culled or
// unseen) skip the coefficient load: their gradients are exactly zero.
constexpr int kShBlock = 64;

// Moves `count` (<= kShBlock) rows of KC floats between global memory
// (contiguous rows) and LDS rows of `Pitch` floats. Every lane issues all of
// its loads before the first LDS write, 16 bytes at a time when Vec (the
// global rows are 16-byte aligned and KC % 4 == 0). stage_rows skips rows
// whose `needs` flag is clear.
template <int KC, int Pitch, bool Vec>
__device__ __forceinline__ void stage_rows(const float* __restrict__ src, float* lds, int count,
                                           const int* needs, int t) {
  if constexpr (Vec && KC % 4 == 0) {
    constexpr int kPer = KC / 4;  // float4 per lane: kShBlock * KC / 4 / kShBlock
    float4 v[kPer];
#pragma unroll
    for (int it = 0; it < kPer; ++it) {
      const int q = it * kShBlock + t;  // float4 index in the block's rows
      const int row = (4 * q) / KC;
      v[it] = (row < count && needs[row]) ? reinterpret_cast<const float4*>(src)[q]
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int it = 0; it < kPer; ++it) {
      const int q = it * kShBlock + t;
      const int row = (4 * q) / KC, k = 4 * q - row * KC;
      float* d = lds + row * Pitch + k;
      if (row < count) {
        d[0] = v[it].x;
        d[1] = v[it].y;
        d[2] = v[it].z;
        d[3] = v[it].w;
      }
    }
  } else {
    float v[KC];
#pragma unroll
    for (int it = 0; it < KC; ++it) {
      const int e = it * kShBlock + t;
      const int row = e / KC;
      v[it] = (row < count && needs[row]) ? src[e] : 0.f;
    }
#pragma unroll
    for (int it = 0; it < KC; ++it) {
      const int e = it * kShBlock + t;
      const int row = e / KC, k = e - row * KC;
      if (row < count) lds[row * Pitch + k] = v[it];
    }
  }
}

template <int KC, int Pitch, bool Vec>
__device__ __forceinline__ void unstage_rows(const float* lds, float* __restrict__ dst, int count,
                                             int t) {
  if constexpr (Vec && KC % 4 == 0) {
#pragma unroll
    for (int it = 0; it < KC / 4; ++it) {
      const int q = it * kShBlock + t;
      const int row = (4 * q) / KC, k = 4 * q - row * KC;
      if (row < count) {
        const float* s = lds + row * Pitch + k;
        reinterpret_cast<float4*>(dst)[q] = make_float4(s[0], s[1], s[2], s[3]);
      }
    }
  } else {
#pragma unroll
    for (int it = 0; it < KC; ++it) {
      const int e = it * kShBlock + t;
      const int row = e / KC, k = e - row * KC;
      if (row < count) dst[e] = lds[row * Pitch + k];
    }
  }
}

// Vec: coefficient arrays and their gradients start on 16-byte boundaries.
// A workgroup of two waves takes kShBlock surfels: wave `set` stages and
// differentiates colour set `set` (first or second coefficients), so each
// lane keeps one set's 3K gradients in registers rather than both - twice
// the waves per CU for the same LDS. The two sets' direction gradients are
// summed through LDS; wave 0 also writes the shared-parameter and opacity
// gradients.
constexpr int kShSets = 2;

template <int Degree, bool Vec>
__global__ __launch_bounds__(kShBlock * kShSets) void sh_rows_backward_kernel(
    const float* __restrict__ sh_first, const float* __restrict__ sh_second, int64_t cameras,
    int64_t n, const int* __restrict__ row_of_pair, const float* __restrict__ geometry,
    const float* __restrict__ grad_rows, const float* __restrict__ grad_opacity_rows,
    float* __restrict__ grad_first, float* __restrict__ grad_second,
    float* __restrict__ grad_weights, float* __restrict__ grad_magnitudes,
    float* __restrict__ grad_phases, float* __restrict__ grad_opacities,
    float* __restrict__ grad_directions) {
  constexpr int K = (Degree + 1) * (Degree + 1);
  constexpr int KC = K * 3;      // floats per surfel and colour set
  constexpr int PITCH = KC + 1;  // odd pitch
  __shared__ float stage[kShSets][kShBlock * PITCH];
  __shared__ int needs[kShBlock];
  __shared__ float set1_directions[kShBlock][3];
  const int t = threadIdx.x & (kShBlock - 1);
  const int set = threadIdx.x / kShBlock;  // uniform per wave
  const int64_t first = int64_t(blockIdx.x) * kShBlock;
  const int64_t scene = blockIdx.y;
  const int count = int(min<int64_t>(kShBlock, n - first));
  const int64_t i = first + t;
  const bool own = t < count;
  const int64_t surfel = scene * n + i;
  // Pass 1 (wave 0): the colour gradients decide whether the coefficients
  // matter.
  if (set == 0) {
    bool any = false;
    if (own) {
      for (int64_t c = 0; c < cameras && !any; ++c) {
        const int64_t pair = (scene * cameras + c) * n + i;
        const int64_t row = row_of_pair ? int64_t(row_of_pair[pair]) : pair;
        if (row < 0) continue;
        const float* gr = grad_rows + row * kRow;
#pragma unroll
        for (int k = 0; k < 6; ++k) any |= gr[k] != 0.f;
      }
    }
    needs[t] = any;
  }
  __syncthreads();
  const int64_t base = (scene * n + first) * KC;
  float* lds = stage[set];
  stage_rows<KC, PITCH, Vec>((set ? sh_second : sh_first) + base, lds, count, needs, t);
  __syncthreads();
  const float* coef = lds + t * PITCH;  // coef[k * 3 + ch]
  float acc[KC];
#pragma unroll
  for (int k = 0; k < KC; ++k) acc[k] = 0.f;
  float shared[12];
#pragma unroll
  for (int k = 0; k < 12; ++k) shared[k] = 0.f;
  float g_opacity = 0.f;
  // Every thread runs every camera (the LDS exchange below needs both
  // waves); lanes past `count` only take part in the barriers.
  for (int64_t c = 0; c < cameras; ++c) {
    // Read the coefficients from LDS where they are used, in every camera:
    // hoisted out of the loop they would hold 3K registers throughout it.
    asm volatile("" ::: "memory");
    const int64_t pair = (scene * cameras + c) * n + i;
    int64_t row = -1;
    if (own) row = row_of_pair ? int64_t(row_of_pair[pair]) : pair;
    float gd[3] = {0.f, 0.f, 0.f};
    if (row >= 0) {
      const float* gr = grad_rows + row * kRow;
      float g[3];
      bool nonzero = false;
#pragma unroll
      for (int ch = 0; ch < 3; ++ch) {
        g[ch] = gr[set * 3 + ch];
        nonzero |= g[ch] != 0.f;
      }
      if (nonzero) {
        // Colours and coefficient gradients from the basis values; the
        // direction gradient sum_k w_k grad(Y_k), w_k = sum_ch gc_ch coef_k,ch,
        // from the basis derivatives afterwards, so that values and
        // derivatives are not live together.
        const float* d = geometry + row * kGeometry + 14;
        float Y[K], w[K];
        sh_basis<Degree, false>(d[0], d[1], d[2], Y, nullptr, nullptr, nullptr);
        float gc[3];
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) {
          float raw = 0.5f;
#pragma unroll
          for (int k = 0; k < K; ++k) raw += Y[k] * coef[k * 3 + ch];
          gc[ch] = raw >= 0.f ? g[ch] : 0.f;
        }
        // The coefficients are read from LDS again below rather than kept
        // in registers across the clamp decisions.
        asm volatile("" ::: "memory");
#pragma unroll
        for (int k = 0; k < K; ++k) {
          w[k] = 0.f;
#pragma unroll
          for (int ch = 0; ch < 3; ++ch) {
            acc[k * 3 + ch] += gc[ch] * Y[k];
            w[k] += gc[ch] * coef[k * 3 + ch];
          }
        }
        float dx[K], dy[K], dz[K];
        sh_basis<Degree, true>(d[0], d[1], d[2], Y, dx, dy, dz);
#pragma unroll
        for (int k = 0; k < K; ++k) {
          gd[0] += w[k] * dx[k];
          gd[1] += w[k] * dy[k];
          gd[2] += w[k] * dz[k];
        }
      }
      if (set == 0) {
#pragma unroll
        for (int k = 0; k < 12; ++k) shared[k] += gr[6 + k];
        if (grad_opacity_rows) g_opacity += grad_opacity_rows[row];
      }
    }
    if (set == 1) {
#pragma unroll
      for (int k = 0; k < 3; ++k) set1_directions[t][k] = gd[k];
    }
    __syncthreads();
    if (set == 0 && row >= 0) {
#pragma unroll
      for (int k = 0; k < 3; ++k) grad_directions[pair * 3 + k] = gd[k] + set1_directions[t][k];
    }
    __syncthreads();  // the next camera overwrites set1_directions
  }
  // Every lane of this wave is done reading its coefficients: the stage
  // takes the gradients.
  float* out = lds + t * PITCH;
#pragma unroll
  for (int k = 0; k < KC; ++k) out[k] = acc[k];
  __syncthreads();
  unstage_rows<KC, PITCH, Vec>(lds, (set ? grad_second : grad_first) + base, count, t);
  if (set == 0 && own) {
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      grad_weights[surfel * 4 + f] = shared[f];
      grad_magnitudes[surfel * 4 + f] = shared[4 + f];
      grad_phases[surfel * 4 + f] = shared[8 + f];
    }
    grad_opacities[surfel] = g_opacity;
  }
}

// Per-pair output gradients read from compositor rows.
struct RowGrads {
  const int* row_of_pair;       // null: row = pair
  const float* geometry;        // [Q,17] dL/d(geometry row), or null
  const float* projected;       // dL/d(projected means), row r at projected + r * stride
  int64_t projected_stride;     // floats between rows of `projected` (2 when contiguous)
  const float* sh_directions;   // [S*C*N,3] direction gradients from SH, or null
  __device__ bool fetch(int64_t pair, PairGrads& g) const {
    const int64_t row = row_of_pair ? int64_t(row_of_pair[pair]) : pair;
    if (row < 0) return false;
    const float* gg = geometry ? geometry + row * kGeometry : nullptr;
#pragma unroll
    for (int k = 0; k < 9; ++k) g.gT[k] = gg ? gg[k] : 0.f;
    // The geometry row's own xy columns duplicate the projected means;
    // their gradient arrives through `projected` only.
    g.has_xy = projected != nullptr;
    g.gxy[0] = projected ? projected[row * projected_stride + 0] : 0.f;
    g.gxy[1] = projected ? projected[row * projected_stride + 1] : 0.f;
    g.has_n = gg != nullptr;
    g.has_d = gg != nullptr || sh_directions != nullptr;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      g.gn[k] = gg ? gg[11 + k] : 0.f;
      g.gd[k] = (gg ? gg[14 + k] : 0.f) + (sh_directions ? sh_directions[pair * 3 + k] : 0.f);
    }
    return true;
  }
};

struct BackwardWorkspace {
  float* partials;
  float* directions;
  size_t bytes;
};

BackwardWorkspace backward_layout(void* base, int64_t scenes, int64_t cameras, int64_t n,
                                  int sh_degree) {
  BackwardWorkspace w;
  char* p = static_cast<char*>(base);
  size_t offset = 0;
  w.partials = reinterpret_cast<float*>(p);
  offset = align_up(camera_partials_bytes(scenes, cameras, n), 256);
  w.directions = sh_degree >= 0 ? reinterpret_cast<float*>(p + offset) : nullptr;
  if (sh_degree >= 0) offset = align_up(offset + size_t(scenes * cameras * n) * 12, 256);
  w.bytes = offset;
  return w;
}

}  // namespace
}  // namespace gs

extern "C" {

int gs_records_forward(const float* means, const float* quaternions, const float* scales,
                       const float* opacities, const float* view_matrices,
                       const float* intrinsics, const float* sh_first, const float* sh_second,
                       const float* frequency_weights, const float* frequency_magnitudes,
                       const float* phases, int32_t sh_degree, int64_t scenes,
                       int64_t cameras, int64_t n, int32_t width, int32_t height,
                       float near_plane, float far_plane, const int32_t* row_of_pair,
                       int32_t* dense_radii, float* geometry, float* projected_means,
                       int32_t* row_radii, int64_t* primitive_ids, int64_t* image_ids,
                       float* appearance_rows, float* opacity_rows, int64_t* meta_scene_ids,
                       int64_t* meta_camera_ids, int64_t* meta_surfel_ids, void* stream) {
  using namespace gs;
  clear_error();
  int status = check_projection_sizes(scenes, cameras, n);
  if (status != GS_OK) return status;
  GS_REQUIRE(width > 0 && height > 0, GS_ERR_ARGUMENT, "invalid image size %dx%d", width, height);
  GS_REQUIRE(sh_degree >= -1 && sh_degree <= 3, GS_ERR_ARGUMENT,
             "SH degree must be -1 (none) or 0 through 3");
  if (n == 0) return GS_OK;
  GS_REQUIRE(means && quaternions && scales && view_matrices && intrinsics, GS_ERR_ARGUMENT,
             "null geometry input passed to gs_records_forward");
  GS_REQUIRE(geometry || dense_radii, GS_ERR_ARGUMENT, "gs_records_forward has no output");
  if (geometry) {
    GS_REQUIRE(projected_means && row_radii && primitive_ids && image_ids, GS_ERR_ARGUMENT,
               "null row output passed to gs_records_forward");
    GS_REQUIRE((meta_scene_ids && meta_camera_ids && meta_surfel_ids) ||
                   (!meta_scene_ids && !meta_camera_ids && !meta_surfel_ids),
               GS_ERR_ARGUMENT, "meta id outputs must be given together");
    if (sh_degree >= 0)
      GS_REQUIRE(opacities && sh_first && sh_second && frequency_weights &&
                     frequency_magnitudes && phases && appearance_rows && opacity_rows,
                 GS_ERR_ARGUMENT, "null SH input or output passed to gs_records_forward");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_PROJECT_FWD, s);
  dim3 grid(static_cast<unsigned>(ceil_div(n, kProjectBlock)), static_cast<unsigned>(scenes));
  const int tw = tiles_x(width), th = tiles_y(height);
  const bool vec = sh_degree < 0 || (aligned16(sh_first) && aligned16(sh_second) &&
                                      aligned16(frequency_weights) &&
                                      aligned16(frequency_magnitudes) && aligned16(phases));
#define GS_RECORDS(D)                                                                        \
  if (vec) GS_RECORDS_V(D, true) else GS_RECORDS_V(D, false)
#define GS_RECORDS_V(D, V)                                                                   \
  records_forward_kernel<D, V><<<grid, kProjectBlock, 0, s>>>(                               \
      means, quaternions, scales, opacities, view_matrices, intrinsics, sh_first, sh_second, \
      frequency_weights, frequency_magnitudes, phases, cameras, n, tw, th, near_plane,      \
      far_plane, row_of_pair, dense_radii, geometry, projected_means, row_radii,             \
      primitive_ids, image_ids, appearance_rows, opacity_rows, meta_scene_ids, meta_camera_ids, \
      meta_surfel_ids);
  switch (sh_degree) {
    case -1: GS_RECORDS(-1); break;
    case 0: GS_RECORDS(0); break;
    case 1: GS_RECORDS(1); break;
    case 2: GS_RECORDS(2); break;
    default: GS_RECORDS(3); break;
  }
#undef GS_RECORDS
#undef GS_RECORDS_V
  GS_LAUNCHED("records_forward_kernel");
  return GS_OK;
}

size_t gs_records_backward_workspace_size(int64_t scenes, int64_t cameras, int64_t n,
                                          int32_t sh_degree) {
  return gs::backward_layout(nullptr, scenes, cameras, n, sh_degree).bytes + 256;
}

int gs_records_backward(const float* means, const float* quaternions, const float* scales,
                        const float* view_matrices, const float* intrinsics,
                        const float* sh_first, const float* sh_second, int32_t sh_degree,
                        int64_t scenes, int64_t cameras, int64_t n,
                        const int32_t* row_of_pair, const float* geometry,
                        const float* grad_geometry, const float* grad_projected_means,
                        int64_t grad_projected_stride, const float* grad_appearance_rows,
                        const float* grad_opacity_rows, float* grad_means, float* grad_quaternions, float* grad_scales,
                        float* grad_view_matrices, float* grad_intrinsics,
                        float* grad_sh_first, float* grad_sh_second, float* grad_weights,
                        float* grad_magnitudes, float* grad_phases, float* grad_opacities,
                        void* workspace, size_t workspace_bytes, void* stream) {
  using namespace gs;
  clear_error();
  int status = check_projection_sizes(scenes, cameras, n);
  if (status != GS_OK) return status;
  GS_REQUIRE(sh_degree >= -1 && sh_degree <= 3, GS_ERR_ARGUMENT,
             "SH degree must be -1 (none) or 0 through 3");
  // Both camera gradient pointers null: the caller's cameras take no
  // gradient, and their adjoint is skipped.
  GS_REQUIRE(!grad_view_matrices == !grad_intrinsics, GS_ERR_ARGUMENT,
             "null camera gradient pointer");
  const bool camera_grads = grad_view_matrices != nullptr;
  GS_REQUIRE(!grad_projected_means || grad_projected_stride >= 2, GS_ERR_ARGUMENT,
             "projected-means gradient rows must be at least 2 floats apart, got %lld",
             static_cast<long long>(grad_projected_stride));
  const size_t need = gs_records_backward_workspace_size(scenes, cameras, n, sh_degree);
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE,
             "record backward needs %zu workspace bytes, got %zu", need, workspace_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_PROJECT_BWD, s);
  BackwardWorkspace w = backward_layout(workspace, scenes, cameras, n, sh_degree);
  const int64_t blocks = ceil_div(n, kProjectBlock);
  if (n > 0) {
    GS_REQUIRE(means && quaternions && scales && view_matrices && intrinsics && grad_means &&
                   grad_quaternions && grad_scales,
               GS_ERR_ARGUMENT, "null pointer passed to gs_records_backward");
    dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(scenes));
    const float* sh_dirs = nullptr;
    if (sh_degree >= 0) {
      GS_REQUIRE(sh_first && sh_second && geometry && grad_appearance_rows && grad_sh_first &&
                     grad_sh_second && grad_weights && grad_magnitudes && grad_phases &&
                     grad_opacities,
                 GS_ERR_ARGUMENT, "null SH pointer passed to gs_records_backward");
      dim3 sh_grid(static_cast<unsigned>(ceil_div(n, kShBlock)), static_cast<unsigned>(scenes));
      const bool vec = aligned16(sh_first) && aligned16(sh_second) &&
                       aligned16(grad_sh_first) && aligned16(grad_sh_second);
#define GS_SH_ROWS(D)                                                                        \
  if (vec) GS_SH_ROWS_V(D, true) else GS_SH_ROWS_V(D, false)
#define GS_SH_ROWS_V(D, V)                                                                   \
  sh_rows_backward_kernel<D, V><<<sh_grid, kShBlock * kShSets, 0, s>>>(                      \
      sh_first, sh_second, cameras, n, row_of_pair, geometry, grad_appearance_rows,          \
      grad_opacity_rows, grad_sh_first, grad_sh_second, grad_weights, grad_magnitudes,       \
      grad_phases, grad_opacities, w.directions);
      switch (sh_degree) {
        case 0: GS_SH_ROWS(0); break;
        case 1: GS_SH_ROWS(1); break;
        case 2: GS_SH_ROWS(2); break;
        default: GS_SH_ROWS(3); break;
      }
#undef GS_SH_ROWS
#undef GS_SH_ROWS_V
      GS_LAUNCHED("sh_rows_backward_kernel");
      sh_dirs = w.directions;
    }
    const RowGrads source{row_of_pair, grad_geometry, grad_projected_means,
                          grad_projected_stride, sh_dirs};
    if (camera_grads)
      projection_backward_kernel<RowGrads, true><<<grid, kProjectBlock, 0, s>>>(
          means, quaternions, scales, view_matrices, intrinsics, cameras, n, source,
          grad_means, grad_quaternions, grad_scales, w.partials);
    else
      projection_backward_kernel<RowGrads, false><<<grid, kProjectBlock, 0, s>>>(
          means, quaternions, scales, view_matrices, intrinsics, cameras, n, source,
          grad_means, grad_quaternions, grad_scales, nullptr);
    GS_LAUNCHED("projection_backward_kernel");
  }
  if (!camera_grads) return GS_OK;
  camera_reduce_kernel<<<static_cast<unsigned>(scenes * cameras), kProjectBlock, 0, s>>>(
      w.partials, blocks, grad_view_matrices, grad_intrinsics);
  GS_LAUNCHED("camera_reduce_kernel");
  return GS_OK;
}

}  // extern "C"
