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

namespace gs {
namespace {

constexpr int kBlock = 256;

// Standard real-SH normalisation constants.
constexpr float kC0 = 0.28209479177387814f;    // 1 / (2 sqrt(pi))
constexpr float kC1 = 0.4886025119029199f;     // sqrt(3 / (4 pi))
constexpr float kC2a = 1.0925484305920792f;    // sqrt(15 / pi) / 2
constexpr float kC2b = 0.31539156525252005f;   // sqrt(5 / pi) / 4
constexpr float kC2c = 0.5462742152960396f;    // sqrt(15 / pi) / 4
constexpr float kC3a = 0.5900435899266435f;    // sqrt(35 / (2 pi)) / 4
constexpr float kC3b = 2.890611442640554f;     // sqrt(105 / pi) / 2
constexpr float kC3c = 0.4570457994644658f;    // sqrt(21 / (2 pi)) / 4
constexpr float kC3d = 0.3731763325901154f;    // sqrt(7 / pi) / 4
constexpr float kC3e = 1.445305721320277f;     // sqrt(105 / pi) / 4

// Basis values Y[k] and, when Grad, their partial derivatives.
template <int Degree, bool Grad>
__device__ __forceinline__ void sh_basis(float x, float y, float z, float* Y, float* dx,
                                         float* dy, float* dz) {
  Y[0] = kC0;
  if constexpr (Grad) dx[0] = dy[0] = dz[0] = 0.f;
  if constexpr (Degree >= 1) {
    Y[1] = -kC1 * y;
    Y[2] = kC1 * z;
    Y[3] = -kC1 * x;
    if constexpr (Grad) {
      dx[1] = 0.f, dy[1] = -kC1, dz[1] = 0.f;
      dx[2] = 0.f, dy[2] = 0.f, dz[2] = kC1;
      dx[3] = -kC1, dy[3] = 0.f, dz[3] = 0.f;
    }
  }
  if constexpr (Degree >= 2) {
    const float xx = x * x, yy = y * y, zz = z * z;
    Y[4] = kC2a * x * y;
    Y[5] = -kC2a * y * z;
    Y[6] = kC2b * (2.f * zz - xx - yy);
    Y[7] = -kC2a * x * z;
    Y[8] = kC2c * (xx - yy);
    if constexpr (Grad) {
      dx[4] = kC2a * y, dy[4] = kC2a * x, dz[4] = 0.f;
      dx[5] = 0.f, dy[5] = -kC2a * z, dz[5] = -kC2a * y;
      dx[6] = -2.f * kC2b * x, dy[6] = -2.f * kC2b * y, dz[6] = 4.f * kC2b * z;
      dx[7] = -kC2a * z, dy[7] = 0.f, dz[7] = -kC2a * x;
      dx[8] = 2.f * kC2c * x, dy[8] = -2.f * kC2c * y, dz[8] = 0.f;
    }
  }
  if constexpr (Degree >= 3) {
    const float xx = x * x, yy = y * y, zz = z * z;
    Y[9] = -kC3a * y * (3.f * xx - yy);
    Y[10] = kC3b * x * y * z;
    Y[11] = -kC3c * y * (4.f * zz - xx - yy);
    Y[12] = kC3d * z * (2.f * zz - 3.f * xx - 3.f * yy);
    Y[13] = -kC3c * x * (4.f * zz - xx - yy);
    Y[14] = kC3e * z * (xx - yy);
    Y[15] = -kC3a * x * (xx - 3.f * yy);
    if constexpr (Grad) {
      dx[9] = -6.f * kC3a * x * y, dy[9] = -3.f * kC3a * (xx - yy), dz[9] = 0.f;
      dx[10] = kC3b * y * z, dy[10] = kC3b * x * z, dz[10] = kC3b * x * y;
      dx[11] = 2.f * kC3c * x * y, dy[11] = -kC3c * (4.f * zz - xx - 3.f * yy);
      dz[11] = -8.f * kC3c * y * z;
      dx[12] = -6.f * kC3d * x * z, dy[12] = -6.f * kC3d * y * z;
      dz[12] = kC3d * (6.f * zz - 3.f * xx - 3.f * yy);
      dx[13] = -kC3c * (4.f * zz - 3.f * xx - yy), dy[13] = 2.f * kC3c * x * y;
      dz[13] = -8.f * kC3c * x * z;
      dx[14] = 2.f * kC3e * x * z, dy[14] = -2.f * kC3e * y * z, dz[14] = kC3e * (xx - yy);
      dx[15] = -3.f * kC3a * (xx - yy), dy[15] = 6.f * kC3a * x * y, dz[15] = 0.f;
    }
  }
}

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
