// Real spherical-harmonic basis (degree 0-3) and its direction derivatives,
// in the ordering and sign convention of the Gaussian-splatting family
// (Y_1 = -C1 y, Y_2 = C1 z, Y_3 = -C1 x, ...); see sh.hip.
#pragma once

#include <hip/hip_runtime.h>

namespace gs {

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

}  // namespace gs
