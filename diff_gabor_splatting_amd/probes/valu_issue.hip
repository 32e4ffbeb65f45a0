// VALU issue-rate probe for gfx950: how many SIMD cycles a wave64 VALU
// instruction takes in chains of fused multiply-adds alone and interleaved
// with transcendentals, DPP adds, plain adds or multiplies. It is a stand-alone
// program (not part of the library), used to read the compositors' VALU
// counters: the single-issue model of one wave64 instruction per SIMD every
// 4 cycles is what the roofline's issue fraction divides by.
//
// Build and run (one GPU):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       diff_gabor_splatting_amd/probes/valu_issue.hip -o /tmp/valu_issue && /tmp/valu_issue
//
// Each lane runs eight independent FMA chains (operands: the chain, one
// SGPR and an inline constant, so no VGPR bank conflicts), 2048 iterations,
// 16 waves per SIMD. Cycles per instruction assume the 2.4 GHz peak clock.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#define CHECK(call)                                                              \
  do {                                                                           \
    hipError_t e_ = (call);                                                      \
    if (e_ != hipSuccess) {                                                      \
      std::fprintf(stderr, "%s: %s\n", #call, hipGetErrorString(e_));            \
      std::exit(1);                                                              \
    }                                                                            \
  } while (0)

constexpr int kIters = 2048;

template <int Mode>
__global__ __launch_bounds__(256) void probe(float* out, float a) {
  float x[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) x[k] = float(threadIdx.x) * 1e-3f + float(k);
  float y = float(threadIdx.x) * 1e-4f;
  for (int i = 0; i < kIters; ++i) {
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = fmaf(x[k], a, 0.5f);
    if constexpr (Mode == 1) y = __builtin_amdgcn_exp2f(y * -0.5f);
    if constexpr (Mode == 2) y = __builtin_amdgcn_sinf(y) + __builtin_amdgcn_cosf(y);
    if constexpr (Mode == 3) {
#pragma unroll
      for (int k = 0; k < 4; ++k) x[k] = __builtin_amdgcn_rcpf(x[k] + 2.f);
    }
    if constexpr (Mode == 4) {  // row_mirror DPP, fused into the add
#pragma unroll
      for (int k = 0; k < 8; ++k)
        x[k] = __builtin_amdgcn_update_dpp(0.f, x[k], 0x140, 0xf, 0xf, false) + x[k];
    }
    if constexpr (Mode == 5) {
#pragma unroll
      for (int k = 0; k < 8; ++k) x[k] = x[k] + x[k];
    }
    if constexpr (Mode == 6) {
#pragma unroll
      for (int k = 0; k < 8; ++k) x[k] = x[k] * x[k];
    }
  }
  float s = y;
#pragma unroll
  for (int k = 0; k < 8; ++k) s += x[k];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// per_iter: VALU instructions per loop iteration in the compiled loop.
template <int Mode>
void run(const char* name, int per_iter, float* out, int blocks) {
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  probe<Mode><<<blocks, 256>>>(out, 0.999f);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  CHECK(hipEventRecord(e0));
  for (int r = 0; r < 5; ++r) probe<Mode><<<blocks, 256>>>(out, 0.999f);
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms = 0;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  ms /= 5;
  const double instr = double(blocks) * 4 * kIters * per_iter;
  std::printf("%-30s %7.3f ms  %.3e wave instructions  %.2f SIMD cycles each at 2.4 GHz\n", name,
              ms, instr, ms * 1e-3 * 2.4e9 * 1024 / instr);
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

int main() {
  const int blocks = 256 * 16;  // 16 waves per SIMD on 256 CUs
  float* out = nullptr;
  CHECK(hipMalloc(&out, size_t(blocks) * 256 * sizeof(float)));
  run<0>("8 FMA", 8, out, blocks);
  run<1>("8 FMA + exp + mul", 10, out, blocks);
  run<2>("8 FMA + sin + cos + add", 11, out, blocks);
  run<3>("8 FMA + 4 rcp + 4 add", 16, out, blocks);
  run<4>("8 FMA + 8 DPP-fused add", 16, out, blocks);
  run<5>("8 FMA + 8 add", 16, out, blocks);
  run<6>("8 FMA + 8 mul", 16, out, blocks);
  CHECK(hipFree(out));
  return 0;
}
