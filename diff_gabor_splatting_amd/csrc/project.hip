// Kernel 1: dense per-(scene, camera, surfel) projection and its adjoint.
//
// The C-ABI twin of the reference's PyTorch projection (src/gabor_splatting/
// rendering.py:176-218): separate transform / xy / normal / direction /
// radius arrays of shape [S, C, N, *]. The renderer itself uses the fused
// record kernels in records.hip, which share this math (projection.hpp).
//
// One thread owns one (scene, surfel) and loops over the cameras of its
// scene: surfel parameters are read once, camera parameters are uniform per
// workgroup, and in the adjoint the surfel gradients are summed over cameras
// in registers (no atomics). Per-camera gradients (view and intrinsics) are
// reduced per workgroup with the wave64 reduce-scatter and summed across
// workgroups by a second deterministic kernel.
#include "projection.hpp"

namespace gs {
namespace {

__global__ __launch_bounds__(kProjectBlock) void project_forward_kernel(
    const float* __restrict__ means, const float* __restrict__ quats,
    const float* __restrict__ scales, const float* __restrict__ views,
    const float* __restrict__ intrinsics, int64_t cameras, int64_t n, int tw, int th,
    float near_plane, float far_plane, float* __restrict__ transform, float* __restrict__ xy,
    float* __restrict__ normals, float* __restrict__ directions, int* __restrict__ radii) {
  const int64_t i = int64_t(blockIdx.x) * kProjectBlock + threadIdx.x;
  const int64_t scene = blockIdx.y;
  if (i >= n) return;
  Surfel s;
  load_surfel(means, quats, scales, scene * n + i, s);
  for (int64_t c = 0; c < cameras; ++c) {
    const int64_t cam = scene * cameras + c;
    Projection p;
    project_pair(s.R, s.mu, s.sc, views + cam * 16, intrinsics + cam * 9, p);
    const int64_t pair = cam * n + i;
#pragma unroll
    for (int k = 0; k < 9; ++k) transform[pair * 9 + k] = p.T[k];
    xy[pair * 2 + 0] = p.xy[0];
    xy[pair * 2 + 1] = p.xy[1];
    const float sign = facing_sign(p);
#pragma unroll
    for (int k = 0; k < 3; ++k) normals[pair * 3 + k] = p.nraw[k] * sign;
    float d[3];
    unit_direction(p, d);
#pragma unroll
    for (int k = 0; k < 3; ++k) directions[pair * 3 + k] = d[k];
    radii[pair] = screen_radius(p, tw, th, near_plane, far_plane);
  }
}

// Output gradients held in separate dense [S, C, N, *] arrays (any may be null).
struct DenseGrads {
  const float* transform;
  const float* xy;
  const float* normals;
  const float* directions;
  __device__ bool fetch(int64_t pair, PairGrads& g) const {
#pragma unroll
    for (int k = 0; k < 9; ++k) g.gT[k] = transform ? transform[pair * 9 + k] : 0.f;
    g.has_xy = xy != nullptr;
    g.has_n = normals != nullptr;
    g.has_d = directions != nullptr;
#pragma unroll
    for (int k = 0; k < 2; ++k) g.gxy[k] = xy ? xy[pair * 2 + k] : 0.f;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      g.gn[k] = normals ? normals[pair * 3 + k] : 0.f;
      g.gd[k] = directions ? directions[pair * 3 + k] : 0.f;
    }
    return true;
  }
};

}  // namespace
}  // namespace gs

extern "C" {

int gs_project_forward(const float* means, const float* quaternions, const float* scales,
                       const float* view_matrices, const float* intrinsics, int64_t scenes,
                       int64_t cameras, int64_t n, int32_t width, int32_t height,
                       float near_plane, float far_plane, float* transform, float* xy,
                       float* normals, float* directions, int32_t* radii, void* stream) {
  using namespace gs;
  clear_error();
  int status = check_projection_sizes(scenes, cameras, n);
  if (status != GS_OK) return status;
  GS_REQUIRE(width > 0 && height > 0, GS_ERR_ARGUMENT, "invalid image size %dx%d", width, height);
  if (n == 0) return GS_OK;
  GS_REQUIRE(means && quaternions && scales && view_matrices && intrinsics && transform && xy &&
                 normals && directions && radii,
             GS_ERR_ARGUMENT, "null pointer passed to gs_project_forward");
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_PROJECT_FWD, s);
  dim3 grid(static_cast<unsigned>(ceil_div(n, kProjectBlock)), static_cast<unsigned>(scenes));
  project_forward_kernel<<<grid, kProjectBlock, 0, s>>>(
      means, quaternions, scales, view_matrices, intrinsics, cameras, n, tiles_x(width),
      tiles_y(height), near_plane, far_plane, transform, xy, normals, directions, radii);
  GS_LAUNCHED("project_forward_kernel");
  return GS_OK;
}

size_t gs_project_backward_workspace_size(int64_t scenes, int64_t cameras, int64_t n) {
  return gs::camera_partials_bytes(scenes, cameras, n);
}

int gs_project_backward(const float* means, const float* quaternions, const float* scales,
                        const float* view_matrices, const float* intrinsics, int64_t scenes,
                        int64_t cameras, int64_t n, const float* grad_transform,
                        const float* grad_xy, const float* grad_normals,
                        const float* grad_directions, float* grad_means,
                        float* grad_quaternions, float* grad_scales,
                        float* grad_view_matrices, float* grad_intrinsics, void* workspace,
                        size_t workspace_bytes, void* stream) {
  using namespace gs;
  clear_error();
  int status = check_projection_sizes(scenes, cameras, n);
  if (status != GS_OK) return status;
  GS_REQUIRE(grad_view_matrices && grad_intrinsics, GS_ERR_ARGUMENT,
             "null camera gradient pointer");
  const size_t need = gs_project_backward_workspace_size(scenes, cameras, n);
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE,
             "projection backward needs %zu workspace bytes, got %zu", need, workspace_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_PROJECT_BWD, s);
  const int64_t blocks = ceil_div(n, kProjectBlock);
  float* partials = static_cast<float*>(workspace);
  if (n > 0) {
    GS_REQUIRE(means && quaternions && scales && view_matrices && intrinsics && grad_means &&
                   grad_quaternions && grad_scales,
               GS_ERR_ARGUMENT, "null pointer passed to gs_project_backward");
    dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(scenes));
    projection_backward_kernel<DenseGrads><<<grid, kProjectBlock, 0, s>>>(
        means, quaternions, scales, view_matrices, intrinsics, cameras, n,
        DenseGrads{grad_transform, grad_xy, grad_normals, grad_directions}, grad_means,
        grad_quaternions, grad_scales, partials);
    GS_LAUNCHED("projection_backward_kernel");
  }
  camera_reduce_kernel<<<static_cast<unsigned>(scenes * cameras), kProjectBlock, 0, s>>>(
      partials, blocks, grad_view_matrices, grad_intrinsics);
  GS_LAUNCHED("camera_reduce_kernel");
  return GS_OK;
}

}  // extern "C"
