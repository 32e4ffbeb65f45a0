// Projection of one (surfel, camera) pair and its adjoint, shared by the
// dense projection op (project.hip) and the fused record kernels
// (records.hip).
//
// Follows the reference's PyTorch projection (src/gabor_splatting/
// rendering.py:156-218): a surfel with unit wxyz quaternion q, tangent
// scales (su, sv) and mean mu maps its local scaled plane to pixels through
// T = K P, P = [Rc R[:,0] su, Rc R[:,1] sv, Rc mu + t]. The conic centre
// and three-sigma extent follow the upstream bound with
// f = [9, 9, -1] / sum([9, 9, -1] * T[2,:]^2).
#pragma once

#include <cmath>

#include "common.hpp"
#include "wave.hpp"

namespace gs {

constexpr int kProjectBlock = 256;
constexpr int kCameraGrads = 21;  // 9 rotation + 3 translation + 9 intrinsics

__device__ __forceinline__ float nan_max(float a, float b) {
  // torch.maximum / amax propagate NaN, fmaxf does not.
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}

__device__ __forceinline__ void quaternion_rotation(float w, float x, float y, float z,
                                                    float R[9]) {
  R[0] = 1.f - 2.f * (y * y + z * z);
  R[1] = 2.f * (x * y - w * z);
  R[2] = 2.f * (x * z + w * y);
  R[3] = 2.f * (x * y + w * z);
  R[4] = 1.f - 2.f * (x * x + z * z);
  R[5] = 2.f * (y * z - w * x);
  R[6] = 2.f * (x * z - w * y);
  R[7] = 2.f * (y * z + w * x);
  R[8] = 1.f - 2.f * (x * x + y * y);
}

// Quantities shared by forward and adjoint for one (surfel, camera).
struct Projection {
  float P[9];     // plane [Rc tu su | Rc tv sv | Rc mu + t], row-major
  float T[9];     // K P
  float D;        // conic denominator
  bool valid;     // D != 0
  float f[3];     // [9, 9, -1] / D (or / 1 when invalid)
  float xy[2];    // conic centre
  float nraw[3];  // Rc R[:,2] before the facing flip
  float facing;
  float dvec[3];  // mu - camera centre
  float dlen;
};

__device__ __forceinline__ void project_pair(const float R[9], const float mu[3],
                                             const float sc[2], const float* V,
                                             const float* K, Projection& p) {
  float Rc[9], t[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
#pragma unroll
    for (int j = 0; j < 3; ++j) Rc[i * 3 + j] = V[i * 4 + j];
    t[i] = V[i * 4 + 3];
  }
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    float c0 = 0.f, c1 = 0.f, c2 = 0.f;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      c0 += Rc[i * 3 + k] * (R[k * 3 + 0] * sc[0]);
      c1 += Rc[i * 3 + k] * (R[k * 3 + 1] * sc[1]);
      c2 += Rc[i * 3 + k] * mu[k];
    }
    p.P[i * 3 + 0] = c0;
    p.P[i * 3 + 1] = c1;
    p.P[i * 3 + 2] = c2 + t[i];
  }
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < 3; ++k) acc += K[i * 3 + k] * p.P[k * 3 + j];
      p.T[i * 3 + j] = acc;
    }
  const float tv[3] = {9.f, 9.f, -1.f};
  p.D = tv[0] * p.T[6] * p.T[6] + tv[1] * p.T[7] * p.T[7] + tv[2] * p.T[8] * p.T[8];
  p.valid = p.D != 0.f;
  const float safe = p.valid ? p.D : 1.f;
#pragma unroll
  for (int k = 0; k < 3; ++k) p.f[k] = tv[k] / safe;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < 3; ++k) acc += p.f[k] * p.T[i * 3 + k] * p.T[6 + k];
    p.xy[i] = acc;
  }
#pragma unroll
  for (int i = 0; i < 3; ++i)
    p.nraw[i] = Rc[i * 3 + 0] * R[2] + Rc[i * 3 + 1] * R[5] + Rc[i * 3 + 2] * R[8];
  p.facing = -(p.P[2] * p.nraw[0] + p.P[5] * p.nraw[1] + p.P[8] * p.nraw[2]);
  // World direction camera centre -> mean; centre = -Rc^T t.
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const float centre = -(Rc[0 * 3 + i] * t[0] + Rc[1 * 3 + i] * t[1] + Rc[2 * 3 + i] * t[2]);
    p.dvec[i] = mu[i] - centre;
  }
  p.dlen = sqrtf(p.dvec[0] * p.dvec[0] + p.dvec[1] * p.dvec[1] + p.dvec[2] * p.dvec[2]);
}

__device__ __forceinline__ float facing_sign(const Projection& p) {
  return p.facing > 0.f ? 1.f : -1.f;
}

__device__ __forceinline__ void unit_direction(const Projection& p, float d[3]) {
  const float inv = 1.f / fmaxf(p.dlen, 1e-12f);
#pragma unroll
  for (int k = 0; k < 3; ++k) d[k] = p.dvec[k] * inv;
}

// Integer screen radius, 0 when culled (rendering.py:207-217): the ceiling of
// the larger three-sigma extent (at least 3*0.707106), visible only for a
// valid conic, a non-edge-on surfel with near < depth < far, finite values
// and a non-empty tile rectangle.
__device__ __forceinline__ int screen_radius(const Projection& p, int tw, int th,
                                             float near_plane, float far_plane) {
  float extent[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    float sq = p.xy[k] * p.xy[k] -
               (p.f[0] * p.T[k * 3 + 0] * p.T[k * 3 + 0] + p.f[1] * p.T[k * 3 + 1] * p.T[k * 3 + 1] +
                p.f[2] * p.T[k * 3 + 2] * p.T[k * 3 + 2]);
    sq = (sq != sq) ? sq : fmaxf(sq, 1e-4f);
    extent[k] = sqrtf(sq);
  }
  const float radius = ceilf(nan_max(nan_max(extent[0], extent[1]), 2.121318f));
  const float fx_tiles = float(tw), fy_tiles = float(th);
  const float lx = fmaxf(truncf((p.xy[0] - radius) / 16.f), 0.f);
  const float ly = fmaxf(truncf((p.xy[1] - radius) / 16.f), 0.f);
  const float ux = fmaxf(truncf((p.xy[0] + radius + 15.f) / 16.f), 0.f);
  const float uy = fmaxf(truncf((p.xy[1] + radius + 15.f) / 16.f), 0.f);
  bool visible = p.valid && p.facing != 0.f && p.P[8] > near_plane && p.P[8] < far_plane;
  visible = visible && isfinite(radius) && radius < 1073741824.f;
  visible = visible && isfinite(p.xy[0]) && isfinite(p.xy[1]);
  visible = visible && fminf(ux, fx_tiles) > fminf(lx, fx_tiles);
  visible = visible && fminf(uy, fy_tiles) > fminf(ly, fy_tiles);
  return visible ? int(radius) : 0;
}

struct Surfel {
  float mu[3], q[4], qn[4], qlen, sc[2], R[9];
};

__device__ __forceinline__ void load_surfel(const float* means, const float* quats,
                                            const float* scales, int64_t i, Surfel& s) {
#pragma unroll
  for (int k = 0; k < 3; ++k) s.mu[k] = means[i * 3 + k];
#pragma unroll
  for (int k = 0; k < 4; ++k) s.q[k] = quats[i * 4 + k];
  s.sc[0] = scales[i * 2 + 0];
  s.sc[1] = scales[i * 2 + 1];
  s.qlen = sqrtf(s.q[0] * s.q[0] + s.q[1] * s.q[1] + s.q[2] * s.q[2] + s.q[3] * s.q[3]);
#pragma unroll
  for (int k = 0; k < 4; ++k) s.qn[k] = s.q[k] / s.qlen;
  quaternion_rotation(s.qn[0], s.qn[1], s.qn[2], s.qn[3], s.R);
}

// A harmless stand-in for lanes past the end (they still join reductions).
__device__ __forceinline__ void idle_surfel(Surfel& s) {
#pragma unroll
  for (int k = 0; k < 3; ++k) s.mu[k] = 0.f;
  s.q[0] = s.qn[0] = 1.f;
  s.q[1] = s.q[2] = s.q[3] = s.qn[1] = s.qn[2] = s.qn[3] = 0.f;
  s.qlen = 1.f;
  s.sc[0] = s.sc[1] = 0.f;
  quaternion_rotation(1.f, 0.f, 0.f, 0.f, s.R);
}

// Output gradients of one pair: transform (always), conic centre, facing
// normal and unit direction (each optional).
struct PairGrads {
  float gT[9], gxy[2], gn[3], gd[3];
  bool has_xy, has_n, has_d;
};

// Adjoint of one pair. Accumulates surfel gradients into gmu, gR (rotation
// matrix) and gs (scales) and the camera's into cam[21] = dRc (9), dt (3),
// dK (9).
__device__ __forceinline__ void pair_adjoint(const Surfel& s, const float* V, const float* K,
                                             const Projection& p, PairGrads& g, float gmu[3],
                                             float gR[9], float gs[2], float cam[kCameraGrads]) {
  float Rc[9], t[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
#pragma unroll
    for (int b = 0; b < 3; ++b) Rc[a * 3 + b] = V[a * 4 + b];
    t[a] = V[a * 4 + 3];
  }
  float* gT = g.gT;
  // Conic centre xy_i = sum_k f_k T_ik T_2k with f = tv / D.
  if (g.has_xy) {
    const float tv[3] = {9.f, 9.f, -1.f};
    float gf[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      gf[k] = 0.f;
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        gT[a * 3 + k] += g.gxy[a] * p.f[k] * p.T[6 + k];
        gT[6 + k] += g.gxy[a] * p.f[k] * p.T[a * 3 + k];
        gf[k] += g.gxy[a] * p.T[a * 3 + k] * p.T[6 + k];
      }
    }
    if (p.valid) {
      // f_k = tv_k / D  =>  dL/dD = -sum_k gf_k f_k / D, D = sum tv_k T_2k^2.
      const float gD = -(gf[0] * p.f[0] + gf[1] * p.f[1] + gf[2] * p.f[2]) / p.D;
#pragma unroll
      for (int k = 0; k < 3; ++k) gT[6 + k] += gD * 2.f * tv[k] * p.T[6 + k];
    }
  }
  // T = K P: dK = gT P^T, dP = K^T gT.
  float gP[9];
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int b = 0; b < 3; ++b) {
      float acc_k = 0.f, acc_p = 0.f;
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        acc_k += gT[a * 3 + k] * p.P[b * 3 + k];
        acc_p += K[k * 3 + a] * gT[k * 3 + b];
      }
      cam[12 + a * 3 + b] += acc_k;
      gP[a * 3 + b] = acc_p;
    }
  float* gRc = cam;
  float* gt = cam + 9;
  // Plane column 2: camera mean Rc mu + t; columns j < 2: Rc (R[:,j] s_j).
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    gt[a] += gP[a * 3 + 2];
#pragma unroll
    for (int b = 0; b < 3; ++b) {
      gRc[a * 3 + b] += gP[a * 3 + 2] * s.mu[b] + gP[a * 3 + 0] * s.R[b * 3 + 0] * s.sc[0] +
                        gP[a * 3 + 1] * s.R[b * 3 + 1] * s.sc[1];
    }
  }
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    float g_mean = 0.f, g_t0 = 0.f, g_t1 = 0.f;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      g_mean += Rc[a * 3 + b] * gP[a * 3 + 2];
      g_t0 += Rc[a * 3 + b] * gP[a * 3 + 0];
      g_t1 += Rc[a * 3 + b] * gP[a * 3 + 1];
    }
    gmu[b] += g_mean;
    gR[b * 3 + 0] += g_t0 * s.sc[0];
    gR[b * 3 + 1] += g_t1 * s.sc[1];
    gs[0] += g_t0 * s.R[b * 3 + 0];
    gs[1] += g_t1 * s.R[b * 3 + 1];
  }
  // Facing normal sign * Rc R[:,2]; the sign is piecewise constant.
  if (g.has_n) {
    const float sign = facing_sign(p);
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      const float gna = sign * g.gn[a];
#pragma unroll
      for (int b = 0; b < 3; ++b) {
        gRc[a * 3 + b] += gna * s.R[b * 3 + 2];
        gR[b * 3 + 2] += Rc[a * 3 + b] * gna;
      }
    }
  }
  // Unit direction d / max(|d|, 1e-12), d = mu + Rc^T t.
  if (g.has_d) {
    float gvec[3];
    if (p.dlen > 1e-12f) {
      const float inv = 1.f / p.dlen;
      const float dot = (p.dvec[0] * g.gd[0] + p.dvec[1] * g.gd[1] + p.dvec[2] * g.gd[2]) * inv;
#pragma unroll
      for (int a = 0; a < 3; ++a) gvec[a] = (g.gd[a] - p.dvec[a] * inv * dot) * inv;
    } else {
#pragma unroll
      for (int a = 0; a < 3; ++a) gvec[a] = g.gd[a] / 1e-12f;
    }
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      gmu[a] += gvec[a];
      // centre = -Rc^T t and d = mu - centre: dt = Rc gvec, dRc = t gvec^T.
      gt[a] += Rc[a * 3 + 0] * gvec[0] + Rc[a * 3 + 1] * gvec[1] + Rc[a * 3 + 2] * gvec[2];
#pragma unroll
      for (int b = 0; b < 3; ++b) gRc[a * 3 + b] += t[a] * gvec[b];
    }
  }
}

// Rotation-matrix gradient -> raw quaternion gradient (through the
// normalisation q / |q|).
__device__ __forceinline__ void quaternion_adjoint(const Surfel& s, const float gR[9],
                                                   float gq_out[4]) {
  const float w = s.qn[0], x = s.qn[1], y = s.qn[2], z = s.qn[3];
  float gq[4];
  gq[0] = 2.f * (-z * gR[1] + y * gR[2] + z * gR[3] - x * gR[5] - y * gR[6] + x * gR[7]);
  gq[1] = 2.f * (y * gR[1] + z * gR[2] + y * gR[3] - 2.f * x * gR[4] - w * gR[5] + z * gR[6] +
                 w * gR[7] - 2.f * x * gR[8]);
  gq[2] = 2.f * (-2.f * y * gR[0] + x * gR[1] + w * gR[2] + x * gR[3] + z * gR[5] - w * gR[6] +
                 z * gR[7] - 2.f * y * gR[8]);
  gq[3] = 2.f * (-2.f * z * gR[0] - w * gR[1] + x * gR[2] + w * gR[3] - 2.f * z * gR[4] +
                 y * gR[5] + x * gR[6] + y * gR[7]);
  const float proj = gq[0] * w + gq[1] * x + gq[2] * y + gq[3] * z;
#pragma unroll
  for (int k = 0; k < 4; ++k) gq_out[k] = (gq[k] - s.qn[k] * proj) / s.qlen;
}

// Kernels get internal linkage: every translation unit that includes this
// header launches its own copy.
namespace {

// Projection adjoint over every (scene, surfel): one thread per surfel loops
// over the cameras of its scene; `Source::fetch(pair, g)` supplies the output
// gradients of a pair (false: the pair carries none). Surfel gradients are
// written once; per-camera gradients are summed per workgroup into
// partials[camera][block][21] for camera_reduce_kernel. Without Cameras the
// camera adjoint, its reduction and the per-camera barriers are compiled
// out and `partials` is not touched (callers whose cameras take no
// gradient).
template <class Source, bool Cameras = true>
__global__ __launch_bounds__(kProjectBlock, 5) void projection_backward_kernel(
    const float* __restrict__ means, const float* __restrict__ quats,
    const float* __restrict__ scales, const float* __restrict__ views,
    const float* __restrict__ intrinsics, int64_t cameras, int64_t n, Source source,
    float* __restrict__ grad_means, float* __restrict__ grad_quats,
    float* __restrict__ grad_scales, float* __restrict__ partials) {
  __shared__ float wave_sums[kProjectBlock / 64][kCameraGrads];
  const int64_t i = int64_t(blockIdx.x) * kProjectBlock + threadIdx.x;
  const int64_t scene = blockIdx.y;
  const bool valid = i < n;
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  Surfel s;
  if (valid) {
    load_surfel(means, quats, scales, scene * n + i, s);
  } else {
    idle_surfel(s);
  }
  float gmu[3] = {0.f, 0.f, 0.f}, gR[9] = {}, gs[2] = {0.f, 0.f};
  for (int64_t c = 0; c < cameras; ++c) {
    const int64_t cam = scene * cameras + c;
    const float* V = views + cam * 16;
    const float* K = intrinsics + cam * 9;
    float cam_grad[kCameraGrads];
#pragma unroll
    for (int k = 0; k < kCameraGrads; ++k) cam_grad[k] = 0.f;
    PairGrads g;
    if (valid && source.fetch(cam * n + i, g)) {
      Projection p;
      project_pair(s.R, s.mu, s.sc, V, K, p);
      pair_adjoint(s, V, K, p, g, gmu, gR, gs, cam_grad);
    }
    if constexpr (Cameras) {
      const float total = wave_reduce_scatter<kCameraGrads>(cam_grad, lane);
      const int param = rs_param<kCameraGrads>(lane);
      if (param < kCameraGrads) wave_sums[wave][param] = total;
      __syncthreads();
      if (threadIdx.x < kCameraGrads) {
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < kProjectBlock / 64; ++w) acc += wave_sums[w][threadIdx.x];
        partials[(cam * gridDim.x + blockIdx.x) * kCameraGrads + threadIdx.x] = acc;
      }
      __syncthreads();
    }
  }
  if (!valid) return;
  float gq[4];
  quaternion_adjoint(s, gR, gq);
  const int64_t idx = scene * n + i;
#pragma unroll
  for (int k = 0; k < 4; ++k) grad_quats[idx * 4 + k] = gq[k];
#pragma unroll
  for (int k = 0; k < 3; ++k) grad_means[idx * 3 + k] = gmu[k];
  grad_scales[idx * 2 + 0] = gs[0];
  grad_scales[idx * 2 + 1] = gs[1];
}

// Sum the per-workgroup camera partials [cams, blocks, 21] into the view
// matrix (rotation + translation, last row zero) and intrinsics gradients.
__global__ __launch_bounds__(kProjectBlock) void camera_reduce_kernel(
    const float* __restrict__ partials, int64_t blocks, float* __restrict__ grad_views,
    float* __restrict__ grad_intrinsics) {
  __shared__ float wave_sums[kProjectBlock / 64][kCameraGrads];
  const int64_t cam = blockIdx.x;
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  float acc[kCameraGrads];
#pragma unroll
  for (int k = 0; k < kCameraGrads; ++k) acc[k] = 0.f;
  for (int64_t b = threadIdx.x; b < blocks; b += kProjectBlock) {
    const float* row = partials + (cam * blocks + b) * kCameraGrads;
#pragma unroll
    for (int k = 0; k < kCameraGrads; ++k) acc[k] += row[k];
  }
  const float total = wave_reduce_scatter<kCameraGrads>(acc, lane);
  const int param = rs_param<kCameraGrads>(lane);
  if (param < kCameraGrads) wave_sums[wave][param] = total;
  __syncthreads();
  if (threadIdx.x < 16) {
    const int r = threadIdx.x / 4, col = threadIdx.x % 4;
    float v = 0.f;
    if (r < 3) {
      const int k = col < 3 ? r * 3 + col : 9 + r;
#pragma unroll
      for (int w = 0; w < kProjectBlock / 64; ++w) v += wave_sums[w][k];
    }
    grad_views[cam * 16 + threadIdx.x] = v;
  } else if (threadIdx.x >= 32 && threadIdx.x < 41) {
    const int k = 12 + threadIdx.x - 32;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kProjectBlock / 64; ++w) v += wave_sums[w][k];
    grad_intrinsics[cam * 9 + threadIdx.x - 32] = v;
  }
}

}  // namespace

inline size_t camera_partials_bytes(int64_t scenes, int64_t cameras, int64_t n) {
  const int64_t blocks = ceil_div(n > 0 ? n : 0, kProjectBlock);
  return size_t(scenes * cameras * blocks * kCameraGrads) * sizeof(float) + 256;
}

inline int check_projection_sizes(int64_t scenes, int64_t cameras, int64_t n) {
  GS_REQUIRE(scenes >= 1 && cameras >= 1 && n >= 0, GS_ERR_ARGUMENT,
             "projection needs scenes >= 1, cameras >= 1, n >= 0 (got %lld, %lld, %lld)",
             (long long)scenes, (long long)cameras, (long long)n);
  GS_REQUIRE(scenes <= 65535, GS_ERR_ARGUMENT, "at most 65535 scenes per call (got %lld)",
             (long long)scenes);
  GS_REQUIRE(scenes * cameras * n <= 0x7fffffffLL, GS_ERR_OVERFLOW,
             "too many (scene, camera, surfel) pairs");
  return GS_OK;
}

}  // namespace gs
