// Kernel 1b: real spherical-harmonic colours (degree 0-3) for both classic
// colour sets, and their adjoint.
//
// Follows the reference's fused SH op (src/gabor_splatting/csrc/
// spherical_harmonics.cu:11-150): colour = max(0.5 + sum_k Y_k(d) c_k, 0)
// with the real SH basis in the ordering and normalisation used by the
// Gaussian-splatting family (Y_1 = -C1 y, Y_2 = C1 z, Y_3 = -C1 x, ...).
// The clamp derivative passes where the raw value is >= 0.
//
// One thread owns one (scene, surfel) and loops over its scene's cameras,
// so the coefficient gradients are summed over cameras in registers and
// written once (the reference uses atomics when C > 1).
#include "common.hpp"
#include "sh_basis.hpp"

namespace gs {
namespace {

constexpr int kBlock = 256;

template <int Degree>
__global__ __launch_bounds__(kBlock) void sh_forward_kernel(
    const float* __restrict__ first, const float* __restrict__ second,
    const float* __restrict__ directions, float* __restrict__ colors, int64_t cameras,
    int64_t n) {
  constexpr int K = (Degree + 1) * (Degree + 1);
  const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t scene = blockIdx.y;
  if (i >= n) return;
  const int64_t surfel = scene * n + i;
  const float* coef[2] = {first + surfel * K * 3, second + surfel * K * 3};
  for (int64_t c = 0; c < cameras; ++c) {
    const int64_t pair = (scene * cameras + c) * n + i;
    float Y[K];
    sh_basis<Degree, false>(directions[pair * 3], directions[pair * 3 + 1],
                            directions[pair * 3 + 2], Y, nullptr, nullptr, nullptr);
#pragma unroll
    for (int set = 0; set < 2; ++set)
#pragma unroll
      for (int ch = 0; ch < 3; ++ch) {
        float raw = 0.5f;
#pragma unroll
        for (int k = 0; k < K; ++k) raw += Y[k] * coef[set][k * 3 + ch];
        colors[pair * 6 + set * 3 + ch] = fmaxf(raw, 0.f);
      }
  }
}

template <int Degree>
__global__ __launch_bounds__(kBlock) void sh_backward_kernel(
    const float* __restrict__ first, const float* __restrict__ second,
    const float* __restrict__ directions, const float* __restrict__ grad_colors,
    float* __restrict__ grad_first, float* __restrict__ grad_second,
    float* __restrict__ grad_directions, int64_t cameras, int64_t n) {
  constexpr int K = (Degree + 1) * (Degree + 1);
  const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t scene = blockIdx.y;
  if (i >= n) return;
  const int64_t surfel = scene * n + i;
  const float* coef[2] = {first + surfel * K * 3, second + surfel * K * 3};
  float* gcoef[2] = {grad_first + surfel * K * 3, grad_second + surfel * K * 3};
  float acc[2][K * 3];
#pragma unroll
  for (int set = 0; set < 2; ++set)
#pragma unroll
    for (int k = 0; k < K * 3; ++k) acc[set][k] = 0.f;
  for (int64_t c = 0; c < cameras; ++c) {
    const int64_t pair = (scene * cameras + c) * n + i;
    float Y[K], dx[K], dy[K], dz[K];
    sh_basis<Degree, true>(directions[pair * 3], directions[pair * 3 + 1],
                           directions[pair * 3 + 2], Y, dx, dy, dz);
    float gd[3] = {0.f, 0.f, 0.f};
#pragma unroll
    for (int set = 0; set < 2; ++set)
#pragma unroll
      for (int ch = 0; ch < 3; ++ch) {
        float raw = 0.5f;
#pragma unroll
        for (int k = 0; k < K; ++k) raw += Y[k] * coef[set][k * 3 + ch];
        const float g = raw >= 0.f ? grad_colors[pair * 6 + set * 3 + ch] : 0.f;
#pragma unroll
        for (int k = 0; k < K; ++k) {
          const float cv = coef[set][k * 3 + ch];
          acc[set][k * 3 + ch] += g * Y[k];
          gd[0] += g * cv * dx[k];
          gd[1] += g * cv * dy[k];
          gd[2] += g * cv * dz[k];
        }
      }
#pragma unroll
    for (int k = 0; k < 3; ++k) grad_directions[pair * 3 + k] = gd[k];
  }
#pragma unroll
  for (int set = 0; set < 2; ++set)
#pragma unroll
    for (int k = 0; k < K * 3; ++k) gcoef[set][k] = acc[set][k];
}

int check_sh(int64_t scenes, int64_t cameras, int64_t n, int degree) {
  GS_REQUIRE(degree >= 0 && degree <= 3, GS_ERR_ARGUMENT, "SH degree must be 0 through 3");
  GS_REQUIRE(scenes >= 1 && cameras >= 1 && n >= 0, GS_ERR_ARGUMENT, "invalid SH sizes");
  GS_REQUIRE(scenes <= 65535, GS_ERR_ARGUMENT, "at most 65535 scenes per call");
  GS_REQUIRE(scenes * cameras * n <= 0x7fffffffLL, GS_ERR_OVERFLOW, "too many SH pairs");
  return GS_OK;
}

}  // namespace
}  // namespace gs

extern "C" {

int gs_sh_forward(const float* first, const float* second, const float* directions,
                  float* colors, int64_t scenes, int64_t cameras, int64_t n, int32_t degree,
                  void* stream) {
  using namespace gs;
  clear_error();
  int status = check_sh(scenes, cameras, n, degree);
  if (status != GS_OK) return status;
  if (n == 0) return GS_OK;
  GS_REQUIRE(first && second && directions && colors, GS_ERR_ARGUMENT,
             "null pointer passed to gs_sh_forward");
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_SH_FWD, s);
  dim3 grid(unsigned(ceil_div(n, kBlock)), unsigned(scenes));
  switch (degree) {
    case 0: sh_forward_kernel<0><<<grid, kBlock, 0, s>>>(first, second, directions, colors, cameras, n); break;
    case 1: sh_forward_kernel<1><<<grid, kBlock, 0, s>>>(first, second, directions, colors, cameras, n); break;
    case 2: sh_forward_kernel<2><<<grid, kBlock, 0, s>>>(first, second, directions, colors, cameras, n); break;
    default: sh_forward_kernel<3><<<grid, kBlock, 0, s>>>(first, second, directions, colors, cameras, n); break;
  }
  GS_LAUNCHED("sh_forward_kernel");
  return GS_OK;
}

int gs_sh_backward(const float* first, const float* second, const float* directions,
                   const float* grad_colors, float* grad_first, float* grad_second,
                   float* grad_directions, int64_t scenes, int64_t cameras, int64_t n,
                   int32_t degree, void* stream) {
  using namespace gs;
  clear_error();
  int status = check_sh(scenes, cameras, n, degree);
  if (status != GS_OK) return status;
  if (n == 0) return GS_OK;
  GS_REQUIRE(first && second && directions && grad_colors && grad_first && grad_second &&
                 grad_directions,
             GS_ERR_ARGUMENT, "null pointer passed to gs_sh_backward");
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_SH_BWD, s);
  dim3 grid(unsigned(ceil_div(n, kBlock)), unsigned(scenes));
#define GS_SH_BWD(D)                                                                      \
  sh_backward_kernel<D><<<grid, kBlock, 0, s>>>(first, second, directions, grad_colors, \
                                                grad_first, grad_second, grad_directions, \
                                                cameras, n)
  switch (degree) {
    case 0: GS_SH_BWD(0); break;
    case 1: GS_SH_BWD(1); break;
    case 2: GS_SH_BWD(2); break;
    default: GS_SH_BWD(3); break;
  }
#undef GS_SH_BWD
  GS_LAUNCHED("sh_backward_kernel");
  return GS_OK;
}

}  // extern "C"
