// Kernels 4 and 5: forward and reverse tile compositors.
//
// Semantics follow the reference compositor (src/gabor_splatting/csrc/
// rasterize.cu:71-399):
//  * per (pixel, record): ray/plane intersection k = x T2 - T0,
//    l = y T2 - T1, p = k x l, (u, v) = p.xy / p.z; upstream low-pass filter
//    rho = min(u^2 + v^2, 2 |xy - pixel|^2); alpha = min(0.99, o exp(-rho/2));
//    records with alpha < 1/255, p.z == 0 or depth < near are skipped;
//  * front-to-back compositing that stops *before* a contribution that
//    would take transmittance below 1e-4, accumulating rgb, depth, normals
//    and the two-moment distortion, then adding T * background;
//  * backward replays each tile in reverse from its largest contributor
//    count, recovering T by division.
//
// MI355X layout: one workgroup of four wave64s per 16x16 tile, each wave
// owning an 8x8 quadrant (compact footprint for divergence). Records are
// gathered into LDS in batches of 64 (geometry | opacity | appearance, 16-B
// aligned rows, read as broadcasts). In the backward, each wave sums its 64
// pixels' gradients with one reduce-scatter (see wave.hpp) and adds them to
// a per-batch LDS accumulator with one ds_add per wave; after the batch the
// workgroup flushes nonzero totals with one global atomic per (tile,
// record, parameter) instead of one per (wave, record, parameter).
#include <climits>
#include <cmath>

#include "common.hpp"
#include "wave.hpp"

namespace gs {
namespace {

constexpr int kBatch = 64;
constexpr float kPi = 3.14159265358979323846f;

// Directions (cos(pi f / 4), sin(pi f / 4)) of the four Gabor frequencies,
// evaluated the way the reference does: float angle pi*f/4, float cos/sin.
__device__ constexpr float kDirX[4] = {1.0f, 0.70710677f, -4.371139e-08f, -0.70710677f};
__device__ constexpr float kDirY[4] = {0.0f, 0.70710677f, 1.0f, 0.70710677f};

template <bool Neural>
struct Layout {
  static constexpr int A = Neural ? kNeural : kClassic;  // appearance floats
  static constexpr int OP = 17;                          // opacity slot in a row
  static constexpr int AP = 18;                          // first appearance slot
  static constexpr int RS = Neural ? 76 : 36;            // LDS row stride (16-B multiple)
  static constexpr int NP = kGeometry + A + 1;           // gradient values per record
};

struct Sample {
  float k[3], l[3], p[3], s[2], depth, e, alpha;
  bool surface;
};

__device__ __forceinline__ void cross3(const float* a, const float* b, float* c) {
  c[0] = a[1] * b[2] - a[2] * b[1];
  c[1] = a[2] * b[0] - a[0] * b[2];
  c[2] = a[0] * b[1] - a[1] * b[0];
}

// Intersect the pixel ray with the surfel plane and evaluate filtered alpha.
template <bool Neural>
__device__ __forceinline__ bool sample_surface(const float* g, float opacity, float x, float y,
                                               float near_plane, Sample& v) {
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    v.k[i] = x * g[6 + i] - g[i];
    v.l[i] = y * g[6 + i] - g[3 + i];
  }
  cross3(v.k, v.l, v.p);
  if (v.p[2] == 0.f) return false;
  v.s[0] = v.p[0] / v.p[2];
  v.s[1] = v.p[1] / v.p[2];
  const float rho3 = v.s[0] * v.s[0] + v.s[1] * v.s[1];
  const float dx = g[9] - x, dy = g[10] - y;
  const float rho2 = 2.f * (dx * dx + dy * dy);
  v.surface = rho3 <= rho2;
  v.depth = (Neural || v.surface) ? v.s[0] * g[6] + v.s[1] * g[7] + g[8] : g[8];
  if (v.depth < near_plane || !isfinite(v.depth)) return false;
  v.e = expf(-0.5f * fminf(rho3, rho2));
  v.alpha = fminf(0.99f, opacity * v.e);
  return v.alpha >= 1.0f / 255.0f;
}

// Classic: two colours mixed by four cosine waves. Neural: 5->6->3 SIREN.
template <bool Neural>
__device__ __forceinline__ void appearance_forward(const float* a, const float* g,
                                                   const Sample& v, float* color,
                                                   float* hidden, float* pre) {
  if constexpr (Neural) {
    const float in[5] = {v.s[0] / 3.f, v.s[1] / 3.f, g[14], g[15], g[16]};
#pragma unroll
    for (int h = 0; h < 6; ++h) {
      float z = a[30 + h];
#pragma unroll
      for (int k = 0; k < 5; ++k) z += a[h * 5 + k] * in[k];
      pre[h] = z;
      hidden[h] = sinf(30.f * z);
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      float z = a[54 + c];
#pragma unroll
      for (int h = 0; h < 6; ++h) z += a[36 + c * 6 + h] * hidden[h];
      color[c] = 1.f / (1.f + expf(-z));
    }
  } else {
    float h1 = 0.f, h2 = 0.f;
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      const float dot = kDirX[f] * v.s[0] + kDirY[f] * v.s[1];
      const float wave = cosf(2.f * kPi * a[10 + f] * dot + a[14 + f]);
      h1 += a[6 + f] * 0.5f * (1.f + wave);
      h2 += a[6 + f] * 0.5f * (1.f - wave);
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) color[c] = h1 * a[c] + h2 * a[3 + c];
  }
}

// Gather `count` records (list positions first, first+step, ...) into LDS.
template <bool Neural>
__device__ __forceinline__ void load_batch(float* rows, int* ids, int64_t* prims, int first,
                                           int step, int count, const int* point_list,
                                           const int64_t* primitive_ids, const float* geometry,
                                           const float* appearance, const float* opacities) {
  using L = Layout<Neural>;
  const int t = threadIdx.x;
  if (t < count) {
    const int id = point_list[first + step * t];
    ids[t] = id;
    prims[t] = primitive_ids[id];
  }
  __syncthreads();
  for (int idx = t; idx < count * L::RS; idx += kTilePixels) {
    const int j = idx / L::RS;
    const int f = idx - j * L::RS;
    float value = 0.f;
    if (f < kGeometry) {
      value = geometry[int64_t(ids[j]) * kGeometry + f];
    } else if (f == L::OP) {
      value = opacities[prims[j]];
    } else if (f - L::AP < L::A) {
      value = appearance[prims[j] * L::A + (f - L::AP)];
    }
    rows[idx] = value;
  }
  __syncthreads();
}

struct TilePixel {
  int image, px, py;
  bool inside;
  int64_t pixel;
};

__device__ __forceinline__ TilePixel tile_pixel(int tile, int width, int height, int tw,
                                                int th) {
  TilePixel t;
  t.image = tile / (tw * th);
  const int local = tile - t.image * (tw * th);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  t.px = (local % tw) * kTile + (wave & 1) * 8 + (lane & 7);
  t.py = (local / tw) * kTile + (wave >> 1) * 8 + (lane >> 3);
  t.inside = t.px < width && t.py < height;
  t.pixel = (int64_t(t.image) * height + t.py) * width + t.px;
  return t;
}

template <bool Neural>
__global__ __launch_bounds__(kTilePixels) void render_forward_kernel(
    int width, int height, int tw, int th, const float* __restrict__ geometry,
    const float* __restrict__ appearance, const float* __restrict__ opacities,
    const int64_t* __restrict__ primitive_ids, const float* __restrict__ backgrounds,
    const int* __restrict__ point_list, const int2* __restrict__ ranges, float near_plane,
    float far_plane, float* __restrict__ maps, float* __restrict__ state,
    int* __restrict__ contributors) {
  using L = Layout<Neural>;
  __shared__ __align__(16) float rows[kBatch * L::RS];
  __shared__ int ids[kBatch];
  __shared__ int64_t prims[kBatch];
  const int tile = blockIdx.x;
  const TilePixel tp = tile_pixel(tile, width, height, tw, th);
  const float x = float(tp.px), y = float(tp.py);
  bool done = !tp.inside;
  float out[kMaps];
#pragma unroll
  for (int c = 0; c < kMaps; ++c) out[c] = 0.f;
  float T = 1.f, m1 = 0.f, m2 = 0.f;
  int last = 0;
  const int2 range = ranges[tile];
  const float mscale = far_plane / (far_plane - near_plane);
  for (int start = range.x; start < range.y; start += kBatch) {
    if (__syncthreads_count(done) == kTilePixels) break;
    const int count = min(kBatch, range.y - start);
    load_batch<Neural>(rows, ids, prims, start, 1, count, point_list, primitive_ids, geometry,
                       appearance, opacities);
    for (int j = 0; j < count && !done; ++j) {
      const float* g = rows + j * L::RS;
      Sample v;
      if (!sample_surface<Neural>(g, g[L::OP], x, y, near_plane, v)) continue;
      const float next = T * (1.f - v.alpha);
      if (next < 0.0001f) {
        done = true;
        break;
      }
      float color[3], hidden[6], pre[6];
      appearance_forward<Neural>(g + L::AP, g, v, color, hidden, pre);
      const float w = T * v.alpha;
      const float m = mscale * (1.f - near_plane / v.depth);
#pragma unroll
      for (int c = 0; c < 3; ++c) {
        out[c] += w * color[c];
        out[5 + c] += w * g[11 + c];
      }
      out[4] += w * v.depth;
      out[8] += w * (m * m * (1.f - T) + m2 - 2.f * m * m1);
      m1 += w * m;
      m2 += w * m * m;
      T = next;
      last = start + j - range.x + 1;
    }
  }
  if (tp.inside) {
#pragma unroll
    for (int c = 0; c < 3; ++c) out[c] += T * backgrounds[tp.image * 3 + c];
    out[3] = 1.f - T;
#pragma unroll
    for (int c = 0; c < kMaps; ++c) maps[tp.pixel * kMaps + c] = out[c];
    state[tp.pixel * 3 + 0] = T;
    state[tp.pixel * 3 + 1] = m1;
    state[tp.pixel * 3 + 2] = m2;
    contributors[tp.pixel] = last;
  }
}

// Appearance adjoint. Classic writes 18 gradients into ga and (u,v)
// gradients into gs; neural writes 57 into ga, (u,v) into gs and the
// direction gradients into gdir.
template <bool Neural>
__device__ __forceinline__ void appearance_backward(const float* a, const float* g,
                                                    const Sample& v, const float* color,
                                                    const float* hidden, const float* pre,
                                                    const float* gc, float* ga, float* gs,
                                                    float* gdir) {
  if constexpr (Neural) {
    const float in[5] = {v.s[0] / 3.f, v.s[1] / 3.f, g[14], g[15], g[16]};
    float gh[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const float gz = gc[c] * color[c] * (1.f - color[c]);
      ga[54 + c] = gz;
#pragma unroll
      for (int h = 0; h < 6; ++h) {
        ga[36 + c * 6 + h] = gz * hidden[h];
        gh[h] += gz * a[36 + c * 6 + h];
      }
    }
    float gi[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < 6; ++h) {
      const float gz = gh[h] * 30.f * cosf(30.f * pre[h]);
      ga[30 + h] = gz;
#pragma unroll
      for (int k = 0; k < 5; ++k) {
        ga[h * 5 + k] = gz * in[k];
        gi[k] += gz * a[h * 5 + k];
      }
    }
    gs[0] += gi[0] / 3.f;
    gs[1] += gi[1] / 3.f;
#pragma unroll
    for (int k = 0; k < 3; ++k) gdir[k] += gi[2 + k];
  } else {
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      const float dot = kDirX[f] * v.s[0] + kDirY[f] * v.s[1];
      const float angle = 2.f * kPi * a[10 + f] * dot + a[14 + f];
      float sn, cs;
      sincosf(angle, &sn, &cs);
      float gw = 0.f, gt = 0.f;
#pragma unroll
      for (int c = 0; c < 3; ++c) {
        ga[c] += gc[c] * a[6 + f] * 0.5f * (1.f + cs);
        ga[3 + c] += gc[c] * a[6 + f] * 0.5f * (1.f - cs);
        gw += gc[c] * 0.5f * ((1.f + cs) * a[c] + (1.f - cs) * a[3 + c]);
        gt += gc[c] * a[6 + f] * 0.5f * sn * (a[3 + c] - a[c]);
      }
      ga[6 + f] += gw;
      ga[10 + f] += gt * 2.f * kPi * dot;
      ga[14 + f] += gt;
      gs[0] += gt * 2.f * kPi * a[10 + f] * kDirX[f];
      gs[1] += gt * 2.f * kPi * a[10 + f] * kDirY[f];
    }
  }
}

template <bool Neural>
__global__ __launch_bounds__(kTilePixels) void render_backward_kernel(
    int width, int height, int tw, int th, const float* __restrict__ geometry,
    const float* __restrict__ appearance, const float* __restrict__ opacities,
    const int64_t* __restrict__ primitive_ids, const float* __restrict__ backgrounds,
    const int* __restrict__ point_list, const int2* __restrict__ ranges,
    const float* __restrict__ state, const int* __restrict__ contributors,
    const float* __restrict__ grad_maps, float near_plane, float far_plane,
    float* __restrict__ grad_geometry, float* __restrict__ grad_appearance,
    float* __restrict__ grad_opacities, float* __restrict__ grad_backgrounds) {
  using L = Layout<Neural>;
  constexpr int NP = L::NP;
  __shared__ __align__(16) float rows[kBatch * L::RS];
  __shared__ float acc[kBatch * NP];
  __shared__ int ids[kBatch];
  __shared__ int64_t prims[kBatch];
  __shared__ int wave_last[4];
  __shared__ float bg_acc[3];
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int tile = blockIdx.x;
  const TilePixel tp = tile_pixel(tile, width, height, tw, th);
  const float x = float(tp.px), y = float(tp.py);
  const int last = tp.inside ? contributors[tp.pixel] : 0;

  for (int i = threadIdx.x; i < kBatch * NP; i += kTilePixels) acc[i] = 0.f;
  if (threadIdx.x < 3) bg_acc[threadIdx.x] = 0.f;
  const int wmax = wave_max(last);
  if (lane == 0) wave_last[wave] = wmax;

  float go[kMaps];
#pragma unroll
  for (int c = 0; c < kMaps; ++c) go[c] = tp.inside ? grad_maps[tp.pixel * kMaps + c] : 0.f;
  const float final_t = tp.inside ? state[tp.pixel * 3 + 0] : 0.f;
  const float m1 = tp.inside ? state[tp.pixel * 3 + 1] : 0.f;
  const float m2 = tp.inside ? state[tp.pixel * 3 + 2] : 0.f;
  const float total_a = 1.f - final_t;
  float T = final_t;
  float background_dot = 0.f;
#pragma unroll
  for (int c = 0; c < 3; ++c) background_dot += go[c] * backgrounds[tp.image * 3 + c];
  __syncthreads();
  // Background gradient: sum over the tile of final T * dL/drgb.
  {
    const float gb[3] = {final_t * go[0], final_t * go[1], final_t * go[2]};
    const float total = wave_reduce_scatter<3>(gb, lane);
    const int param = rs_param<3>(lane);
    if (param < 3 && total != 0.f) atomicAdd(&bg_acc[param], total);
  }
  const int block_last = max(max(wave_last[0], wave_last[1]), max(wave_last[2], wave_last[3]));
  const int2 range = ranges[tile];
  const float mscale = far_plane / (far_plane - near_plane);
  float suffix = 0.f;

  for (int start = block_last; start > 0; start -= kBatch) {
    const int count = min(kBatch, start);
    load_batch<Neural>(rows, ids, prims, range.x + start - 1, -1, count, point_list,
                       primitive_ids, geometry, appearance, opacities);
    for (int j = 0; j < count; ++j) {
      const float* g = rows + j * L::RS;
      const float opacity = g[L::OP];
      Sample v;
      bool active = tp.inside && (start - j) <= last;
      if (active) active = sample_surface<Neural>(g, opacity, x, y, near_plane, v);
      if (!__any(active)) continue;
      float grad[NP];  // geometry 17 | appearance A | opacity
#pragma unroll
      for (int k = 0; k < NP; ++k) grad[k] = 0.f;
      if (active) {
        float* gg = grad;
        float* ga = grad + kGeometry;
        T /= 1.f - v.alpha;
        const float w = T * v.alpha;
        float color[3], hidden[6], pre[6];
        appearance_forward<Neural>(g + L::AP, g, v, color, hidden, pre);
        const float m = mscale * (1.f - near_plane / v.depth);
        float gw = go[4] * v.depth + go[8] * (m * m * total_a + m2 - 2.f * m * m1);
        float gc[3];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          gw += go[c] * color[c] + go[5 + c] * g[11 + c];
          gc[c] = w * go[c];
          gg[11 + c] += w * go[5 + c];
        }
        const float one_minus = 1.f - v.alpha;
        const float galpha =
            T * gw - suffix / one_minus + final_t * (go[3] - background_dot) / one_minus;
        suffix += w * gw;
        float gs[2] = {0.f, 0.f};
        appearance_backward<Neural>(g + L::AP, g, v, color, hidden, pre, gc, ga, gs, gg + 14);
        const float gz = w * go[4] + go[8] * 2.f * w * (m * total_a - m1) * mscale * near_plane /
                                         (v.depth * v.depth);
        if (Neural || v.surface) {
          gs[0] += gz * g[6];
          gs[1] += gz * g[7];
          gg[6] += gz * v.s[0];
          gg[7] += gz * v.s[1];
        }
        gg[8] += gz;
        float grho = 0.f;
        if (opacity * v.e < 0.99f) {
          grad[NP - 1] = galpha * v.e;
          grho = -0.5f * galpha * opacity * v.e;
        }
        if (v.surface) {
          gs[0] += 2.f * v.s[0] * grho;
          gs[1] += 2.f * v.s[1] * grho;
        } else {
          gg[9] += 4.f * (g[9] - x) * grho;
          gg[10] += 4.f * (g[10] - y) * grho;
        }
        const float gp[3] = {gs[0] / v.p[2], gs[1] / v.p[2],
                             -(gs[0] * v.s[0] + gs[1] * v.s[1]) / v.p[2]};
        float gk[3], gl[3];
        cross3(v.l, gp, gk);
        cross3(gp, v.k, gl);
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          gg[k] -= gk[k];
          gg[3 + k] -= gl[k];
          gg[6 + k] += x * gk[k] + y * gl[k];
        }
      }
      // Wave totals, one per lane, added into the batch accumulator.
      float* dst = acc + j * NP;
      if constexpr (NP <= 64) {
        const float total = wave_reduce_scatter<NP>(grad, lane);
        const int param = rs_param<NP>(lane);
        if (param < NP && total != 0.f) atomicAdd(dst + param, total);
      } else {
        constexpr int H = NP / 2;
        float lo[H], hi[NP - H];
#pragma unroll
        for (int k = 0; k < H; ++k) lo[k] = grad[k];
#pragma unroll
        for (int k = 0; k < NP - H; ++k) hi[k] = grad[H + k];
        const float t0 = wave_reduce_scatter<H>(lo, lane);
        const int p0 = rs_param<H>(lane);
        if (p0 < H && t0 != 0.f) atomicAdd(dst + p0, t0);
        const float t1 = wave_reduce_scatter<NP - H>(hi, lane);
        const int p1 = rs_param<NP - H>(lane);
        if (p1 < NP - H && t1 != 0.f) atomicAdd(dst + H + p1, t1);
      }
    }
    __syncthreads();
    // Flush this batch: one global atomic per nonzero (record, parameter).
    for (int idx = threadIdx.x; idx < count * NP; idx += kTilePixels) {
      const float value = acc[idx];
      if (value != 0.f) {
        const int j = idx / NP;
        const int p = idx - j * NP;
        if (p < kGeometry) {
          atomicAdd(grad_geometry + int64_t(ids[j]) * kGeometry + p, value);
        } else if (p < kGeometry + L::A) {
          atomicAdd(grad_appearance + prims[j] * L::A + (p - kGeometry), value);
        } else {
          atomicAdd(grad_opacities + prims[j], value);
        }
        acc[idx] = 0.f;
      }
    }
    // The next batch overwrites ids/prims/rows; every flush must finish first.
    __syncthreads();
  }
  __syncthreads();
  if (threadIdx.x < 3 && bg_acc[threadIdx.x] != 0.f)
    atomicAdd(grad_backgrounds + tp.image * 3 + threadIdx.x, bg_acc[threadIdx.x]);
}

int check_render(int64_t images, int width, int height, float near_plane, float far_plane) {
  GS_REQUIRE(width > 0 && height > 0 && width < INT_MAX - kTile && height < INT_MAX - kTile,
             GS_ERR_ARGUMENT, "invalid image dimensions");
  GS_REQUIRE(near_plane > 0.f && far_plane > near_plane, GS_ERR_ARGUMENT,
             "invalid clipping planes");
  GS_REQUIRE(images >= 1, GS_ERR_ARGUMENT, "invalid backgrounds");
  GS_REQUIRE(images * tiles_x(width) * tiles_y(height) <= INT_MAX, GS_ERR_OVERFLOW,
             "image tile count exceeds int32");
  return GS_OK;
}

}  // namespace
}  // namespace gs

extern "C" {

int gs_render_forward(int32_t neural, const float* geometry, const float* appearance,
                      const float* opacities, const int64_t* primitive_ids,
                      const float* backgrounds, const int32_t* point_list,
                      const int32_t* ranges, int64_t images, int32_t width, int32_t height,
                      float near_plane, float far_plane, float* maps, float* state,
                      int32_t* contributors, void* stream) {
  using namespace gs;
  clear_error();
  int status = check_render(images, width, height, near_plane, far_plane);
  if (status != GS_OK) return status;
  GS_REQUIRE(backgrounds && ranges && maps && state && contributors, GS_ERR_ARGUMENT,
             "null pointer passed to gs_render_forward");
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_RENDER_FWD, s);
  const int tw = tiles_x(width), th = tiles_y(height);
  const unsigned blocks = unsigned(images * tw * th);
  const int2* r = reinterpret_cast<const int2*>(ranges);
  if (neural) {
    render_forward_kernel<true><<<blocks, kTilePixels, 0, s>>>(
        width, height, tw, th, geometry, appearance, opacities, primitive_ids, backgrounds,
        point_list, r, near_plane, far_plane, maps, state, contributors);
  } else {
    render_forward_kernel<false><<<blocks, kTilePixels, 0, s>>>(
        width, height, tw, th, geometry, appearance, opacities, primitive_ids, backgrounds,
        point_list, r, near_plane, far_plane, maps, state, contributors);
  }
  GS_LAUNCHED("render_forward_kernel");
  return GS_OK;
}

int gs_render_backward(int32_t neural, const float* geometry, const float* appearance,
                       const float* opacities, const int64_t* primitive_ids,
                       const float* backgrounds, const int32_t* point_list,
                       const int32_t* ranges, const float* state,
                       const int32_t* contributors, const float* grad_maps, int64_t images,
                       int32_t width, int32_t height, float near_plane, float far_plane,
                       float* grad_geometry, float* grad_appearance, float* grad_opacities,
                       float* grad_backgrounds, void* stream) {
  using namespace gs;
  clear_error();
  int status = check_render(images, width, height, near_plane, far_plane);
  if (status != GS_OK) return status;
  GS_REQUIRE(backgrounds && ranges && state && contributors && grad_maps && grad_backgrounds,
             GS_ERR_ARGUMENT, "null pointer passed to gs_render_backward");
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_RENDER_BWD, s);
  const int tw = tiles_x(width), th = tiles_y(height);
  const unsigned blocks = unsigned(images * tw * th);
  const int2* r = reinterpret_cast<const int2*>(ranges);
  if (neural) {
    render_backward_kernel<true><<<blocks, kTilePixels, 0, s>>>(
        width, height, tw, th, geometry, appearance, opacities, primitive_ids, backgrounds,
        point_list, r, state, contributors, grad_maps, near_plane, far_plane, grad_geometry,
        grad_appearance, grad_opacities, grad_backgrounds);
  } else {
    render_backward_kernel<false><<<blocks, kTilePixels, 0, s>>>(
        width, height, tw, th, geometry, appearance, opacities, primitive_ids, backgrounds,
        point_list, r, state, contributors, grad_maps, near_plane, far_plane, grad_geometry,
        grad_appearance, grad_opacities, grad_backgrounds);
  }
  GS_LAUNCHED("render_backward_kernel");
  return GS_OK;
}

}  // extern "C"
