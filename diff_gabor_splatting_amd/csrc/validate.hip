// Value contracts of the renderer's inputs in one pass over them.
//
// The reference evaluates every contract of check_values
// (src/gabor_splatting/rendering.py:88-153) as its own chain of PyTorch ops
// (isfinite/all per tensor, isclose, a batched matmul, an LU determinant) and
// reads the stacked verdicts back once. Here one kernel reads each input
// once, evaluates every contract on the elements it owns and ORs the
// violated contracts into one 32-bit word (cleared by a one-thread kernel
// first); the caller reads that word back when it chooses.
//
// The launch is a flat list of blocks split into jobs: job 0 checks the
// per-surfel contracts, job 1 the per-image (camera) contracts and jobs
// 2.. the finiteness of each listed tensor. Job boundaries are block
// offsets passed by value, so every block finds its job with a handful of
// scalar compares and the grid holds no empty blocks.
//
// Tolerances follow torch.isclose on float32 operands:
// |x - t| <= atol + |rtol * t|, false for NaN and infinities.

#include "common.hpp"

namespace gs {
namespace {

constexpr int kCheckThreads = 256;
constexpr int kFinitePerThread = 8;
constexpr int64_t kFiniteChunk = int64_t(kCheckThreads) * kFinitePerThread;
constexpr int kJobs = 2 + GS_CHECK_MAX_TENSORS;

struct CheckJobs {
  int64_t first_block[kJobs + 1];  // nondecreasing block offsets; [kJobs] = grid size
  const float* data[GS_CHECK_MAX_TENSORS];
  int64_t count[GS_CHECK_MAX_TENSORS];
  const float* quaternions;
  const float* scales;
  const float* opacities;
  const float* weights;     // null: no frequency-weight contracts (neural)
  const float* magnitudes;  // null: no frequency-magnitude contracts (neural)
  int64_t surfels;
  const float* views;
  const float* intrinsics;
  int64_t images;
};

__device__ __forceinline__ bool close_to(float x, float target, float atol, float rtol) {
  return fabsf(x - target) <= atol + fabsf(rtol * target);
}

// torch.isclose defaults (rtol 1e-5, atol 1e-8) and the unit tolerance of
// the norm, orthonormality, determinant and weight-sum contracts (1e-4).
__device__ __forceinline__ bool exact(float x, float target) {
  return close_to(x, target, 1e-8f, 1e-5f);
}
__device__ __forceinline__ bool unit(float x, float target) {
  return close_to(x, target, 1e-4f, 1e-4f);
}

__device__ uint32_t check_surfel(const CheckJobs& j, int64_t i) {
  uint32_t bad = 0;
  const float s0 = j.scales[2 * i], s1 = j.scales[2 * i + 1];
  if (!(s0 > 0.f && s1 > 0.f)) bad |= GS_CHECK_SCALES_POSITIVE;
  const float o = j.opacities[i];
  if (!(o >= 0.f && o <= 1.f)) bad |= GS_CHECK_OPACITIES_RANGE;
  const float* q = j.quaternions + 4 * i;
  const float norm = ((q[0] * q[0] + q[1] * q[1]) + q[2] * q[2]) + q[3] * q[3];
  if (!unit(norm, 1.f)) bad |= GS_CHECK_QUATERNIONS_UNIT;
  if (j.weights) {
    const float* w = j.weights + 4 * i;
    if (!(w[0] >= 0.f && w[1] >= 0.f && w[2] >= 0.f && w[3] >= 0.f))
      bad |= GS_CHECK_WEIGHTS_NONNEGATIVE;
    if (!unit(((w[0] + w[1]) + w[2]) + w[3], 1.f)) bad |= GS_CHECK_WEIGHTS_SUM;
  }
  if (j.magnitudes) {
    const float* m = j.magnitudes + 4 * i;
    if (!(m[0] >= 0.f && m[1] >= 0.f && m[2] >= 0.f && m[3] >= 0.f))
      bad |= GS_CHECK_MAGNITUDES_NONNEGATIVE;
  }
  return bad;
}

__device__ uint32_t check_image(const CheckJobs& j, int64_t i) {
  uint32_t bad = 0;
  float v[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) v[k] = j.views[16 * i + k];
  if (!(exact(v[12], 0.f) && exact(v[13], 0.f) && exact(v[14], 0.f) && exact(v[15], 1.f)))
    bad |= GS_CHECK_VIEW_LAST_ROW;
  // R^T R against the identity, entry by entry.
  bool orthonormal = true;
#pragma unroll
  for (int a = 0; a < 3; ++a) {
#pragma unroll
    for (int b = 0; b < 3; ++b) {
      const float dot = fmaf(v[8 + a], v[8 + b], fmaf(v[4 + a], v[4 + b], v[a] * v[b]));
      orthonormal = orthonormal && unit(dot, a == b ? 1.f : 0.f);
    }
  }
  if (!orthonormal) bad |= GS_CHECK_ROTATION_ORTHONORMAL;
  const float det = v[0] * (v[5] * v[10] - v[6] * v[9]) - v[1] * (v[4] * v[10] - v[6] * v[8]) +
                    v[2] * (v[4] * v[9] - v[5] * v[8]);
  if (!unit(det, 1.f)) bad |= GS_CHECK_ROTATION_DETERMINANT;
  const float* K = j.intrinsics + 9 * i;
  if (!(exact(K[6], 0.f) && exact(K[7], 0.f) && exact(K[8], 1.f)))
    bad |= GS_CHECK_INTRINSICS_LAST_ROW;
  if (!(K[0] > 0.f && K[4] > 0.f)) bad |= GS_CHECK_FOCAL_POSITIVE;
  return bad;
}

__global__ __launch_bounds__(kCheckThreads) void check_values_kernel(CheckJobs jobs,
                                                                     uint32_t* violations) {
  const int64_t block = blockIdx.x;
  // The job is the last one whose first block is <= this block (empty jobs
  // share their successor's offset and are skipped).
  int job = 0;
#pragma unroll
  for (int k = 1; k < kJobs; ++k) job += block >= jobs.first_block[k] ? 1 : 0;
  const int64_t local = block - jobs.first_block[0];
  uint32_t bad = 0;
  if (job == 0) {
    const int64_t i = local * kCheckThreads + threadIdx.x;
    if (i < jobs.surfels) bad = check_surfel(jobs, i);
  } else if (job == 1) {
    const int64_t i = (block - jobs.first_block[1]) * kCheckThreads + threadIdx.x;
    if (i < jobs.images) bad = check_image(jobs, i);
  } else {
    const float* data = nullptr;
    int64_t count = 0, first = 0;
#pragma unroll
    for (int k = 0; k < GS_CHECK_MAX_TENSORS; ++k) {
      if (job == k + 2) {
        data = jobs.data[k];
        count = jobs.count[k];
        first = jobs.first_block[k + 2];
      }
    }
    const int64_t base = (block - first) * kFiniteChunk + threadIdx.x;
    bool finite = true;
#pragma unroll
    for (int k = 0; k < kFinitePerThread; ++k) {
      const int64_t i = base + int64_t(k) * kCheckThreads;
      if (i < count) finite = finite && isfinite(data[i]);
    }
    if (!finite) bad = 1u << (job - 2);
  }
  // Valid inputs take only the ballot; a violating wave ORs its lanes'
  // words together and publishes them with one atomic.
  if (__any(bad != 0)) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) bad |= __shfl_xor(bad, offset);
    if (__lane_id() == 0) atomicOr(violations, bad);
  }
}

// A kernel rather than a memset, so that the checks can run inside a
// captured HIP graph.
__global__ __launch_bounds__(64) void clear_violations_kernel(uint32_t* violations) {
  if (threadIdx.x == 0) *violations = 0u;
}

}  // namespace
}  // namespace gs

extern "C" {

int gs_check_values(const float* const* tensors, const int64_t* sizes, int32_t tensor_count,
                    const float* quaternions, const float* scales, const float* opacities,
                    const float* frequency_weights, const float* frequency_magnitudes,
                    int64_t surfels, const float* view_matrices, const float* intrinsics,
                    int64_t images, uint32_t* violations, void* stream) {
  using namespace gs;
  clear_error();
  GS_REQUIRE(tensor_count >= 0 && tensor_count <= GS_CHECK_MAX_TENSORS, GS_ERR_ARGUMENT,
             "between 0 and %d tensors can be checked, got %d", GS_CHECK_MAX_TENSORS,
             tensor_count);
  GS_REQUIRE(surfels >= 0 && images >= 0, GS_ERR_ARGUMENT, "negative surfel or image count");
  GS_REQUIRE(violations, GS_ERR_ARGUMENT, "null violations word");
  GS_REQUIRE(tensor_count == 0 || (tensors && sizes), GS_ERR_ARGUMENT, "null tensor list");
  GS_REQUIRE(surfels == 0 || (quaternions && scales && opacities), GS_ERR_ARGUMENT,
             "null surfel tensor passed to gs_check_values");
  GS_REQUIRE(images == 0 || (view_matrices && intrinsics), GS_ERR_ARGUMENT,
             "null camera tensor passed to gs_check_values");
  CheckJobs jobs{};
  int64_t blocks = 0;
  jobs.first_block[0] = blocks;
  blocks += ceil_div(surfels, kCheckThreads);
  jobs.first_block[1] = blocks;
  blocks += ceil_div(images, kCheckThreads);
  for (int k = 0; k < GS_CHECK_MAX_TENSORS; ++k) {
    jobs.first_block[k + 2] = blocks;
    if (k < tensor_count) {
      GS_REQUIRE(sizes[k] >= 0, GS_ERR_ARGUMENT, "negative size of tensor %d", k);
      GS_REQUIRE(sizes[k] == 0 || tensors[k], GS_ERR_ARGUMENT, "null tensor %d", k);
      jobs.data[k] = tensors[k];
      jobs.count[k] = sizes[k];
      blocks += ceil_div(sizes[k], kFiniteChunk);
    }
  }
  jobs.first_block[kJobs] = blocks;
  GS_REQUIRE(blocks <= INT_MAX, GS_ERR_OVERFLOW, "too many values to check");
  jobs.quaternions = quaternions;
  jobs.scales = scales;
  jobs.opacities = opacities;
  jobs.weights = frequency_weights;
  jobs.magnitudes = frequency_magnitudes;
  jobs.surfels = surfels;
  jobs.views = view_matrices;
  jobs.intrinsics = intrinsics;
  jobs.images = images;
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_VALIDATE, s);
  clear_violations_kernel<<<1, 64, 0, s>>>(violations);
  GS_LAUNCHED("clear_violations_kernel");
  if (blocks == 0) return GS_OK;
  check_values_kernel<<<unsigned(blocks), kCheckThreads, 0, s>>>(jobs, violations);
  GS_LAUNCHED("check_values_kernel");
  return GS_OK;
}

}  // extern "C"
