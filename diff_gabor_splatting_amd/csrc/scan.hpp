// Reduce-then-scan over a computed sequence.
//
// A `Load` functor produces item i (so counts can be computed on the fly
// instead of being stored), and a `Store` functor consumes (i, inclusive
// prefix, item). Pass 1 reduces each span, pass 2 exclusive-scans the span
// totals in one workgroup, pass 3 rescans each span with its offset. No
// workgroup waits on another, so there is no inter-block spin.
//
// The span length adapts to the sequence: 256 threads x `rounds` items,
// with rounds chosen so that there are at most about kScanMaxSpans spans.
// Short sequences (radix-sort histograms of a few 10^4 counts) thus get
// many small workgroups, whose latency - not bandwidth - bounds the scan,
// and long ones few enough spans for the single-workgroup pass 2.
#pragma once

#include "common.hpp"

namespace gs {

constexpr int kScanBlock = 256;
constexpr int kScanMinRounds = 2;
constexpr int64_t kScanMaxSpans = 1024;

template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v) {
  const int lane = __lane_id();
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const T up = __shfl_up(v, d, 64);
    if (lane >= d) v += up;
  }
  return v;
}

template <typename T>
__device__ __forceinline__ T block_sum(T v, T* scratch /* >= 4 */) {
  const int lane = __lane_id(), wave = threadIdx.x >> 6;
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  T total = scratch[0] + scratch[1] + scratch[2] + scratch[3];
  __syncthreads();
  return total;
}

template <typename T, typename Load>
__global__ __launch_bounds__(kScanBlock) void scan_reduce_kernel(int64_t count, int rounds,
                                                                 Load load,
                                                                 T* __restrict__ span_sums) {
  __shared__ T scratch[4];
  const int64_t base = int64_t(blockIdx.x) * kScanBlock * rounds;
  T acc = 0;
#pragma unroll 4
  for (int r = 0; r < rounds; ++r) {
    const int64_t i = base + int64_t(r) * kScanBlock + threadIdx.x;
    if (i < count) acc += load(i);
  }
  const T total = block_sum(acc, scratch);
  if (threadIdx.x == 0) span_sums[blockIdx.x] = total;
}

// Exclusive scan of span_sums[0..spans) in place, one workgroup.
template <typename T>
__global__ __launch_bounds__(kScanBlock) void scan_spans_kernel(T* __restrict__ span_sums,
                                                                int64_t spans) {
  __shared__ T totals[2][4];
  const int lane = __lane_id(), wave = threadIdx.x >> 6;
  T carry = 0;
  int parity = 0;
  for (int64_t base = 0; base < spans; base += kScanBlock, parity ^= 1) {
    const int64_t i = base + threadIdx.x;
    const T v = i < spans ? span_sums[i] : T(0);
    const T incl = wave_inclusive_scan(v);
    if (lane == 63) totals[parity][wave] = incl;
    __syncthreads();
    T before = carry;
    for (int w = 0; w < wave; ++w) before += totals[parity][w];
    if (i < spans) span_sums[i] = before + incl - v;
    carry += totals[parity][0] + totals[parity][1] + totals[parity][2] + totals[parity][3];
  }
}

template <typename T, typename Load, typename Store>
__global__ __launch_bounds__(kScanBlock) void scan_down_kernel(int64_t count, int rounds,
                                                               Load load,
                                                               const T* __restrict__ span_offsets,
                                                               Store store) {
  __shared__ T totals[2][4];
  const int lane = __lane_id(), wave = threadIdx.x >> 6;
  const int64_t base = int64_t(blockIdx.x) * kScanBlock * rounds;
  T carry = span_offsets[blockIdx.x];
  for (int r = 0; r < rounds; ++r) {
    const int64_t i = base + int64_t(r) * kScanBlock + threadIdx.x;
    if (base + int64_t(r) * kScanBlock >= count) break;  // uniform across the workgroup
    const T v = i < count ? load(i) : T(0);
    const T incl = wave_inclusive_scan(v);
    if (lane == 63) totals[r & 1][wave] = incl;
    __syncthreads();
    T before = carry;
    for (int w = 0; w < wave; ++w) before += totals[r & 1][w];
    if (i < count) store(i, before + incl, v);
    carry += totals[r & 1][0] + totals[r & 1][1] + totals[r & 1][2] + totals[r & 1][3];
  }
}

// Short sequences (up to kScanLocalItems): one workgroup walks the whole
// sequence in rounds of kScanLocalBlock items, carrying the prefix - one
// launch instead of three.
constexpr int kScanLocalBlock = 1024;
constexpr int64_t kScanLocalItems = 8192;

template <typename T, typename Load, typename Store>
__global__ __launch_bounds__(kScanLocalBlock) void scan_local_kernel(int64_t count, Load load,
                                                                     Store store) {
  constexpr int kWaves = kScanLocalBlock / 64;
  __shared__ T totals[2][kWaves];
  const int lane = __lane_id(), wave = threadIdx.x >> 6;
  T carry = 0;
  int parity = 0;
  for (int64_t base = 0; base < count; base += kScanLocalBlock, parity ^= 1) {
    const int64_t i = base + threadIdx.x;
    const T v = i < count ? load(i) : T(0);
    const T incl = wave_inclusive_scan(v);
    if (lane == 63) totals[parity][wave] = incl;
    __syncthreads();
    T before = carry;
    for (int w = 0; w < wave; ++w) before += totals[parity][w];
    if (i < count) store(i, before + incl, v);
#pragma unroll
    for (int w = 0; w < kWaves; ++w) carry += totals[parity][w];
  }
}

// Items per thread of one span for a sequence of `count` items.
inline int scan_rounds(int64_t count) {
  const int64_t per_span = ceil_div(count > 0 ? count : 0, kScanMaxSpans);
  const int64_t rounds = ceil_div(per_span, kScanBlock);
  return int(rounds < kScanMinRounds ? kScanMinRounds : rounds);
}

inline int64_t scan_spans(int64_t count) {
  return ceil_div(count > 0 ? count : 0, int64_t(kScanBlock) * scan_rounds(count));
}

inline size_t scan_workspace_bytes(int64_t count, size_t item_bytes) {
  return align_up(size_t(scan_spans(count)) * item_bytes, 256) + 256;
}

// Runs the three passes (or, for short sequences, the one-workgroup scan);
// span_sums needs scan_spans(count) entries.
template <typename T, typename Load, typename Store>
int run_scan(int64_t count, Load load, Store store, T* span_sums, hipStream_t stream) {
  if (count <= 0) return GS_OK;
  if (count <= kScanLocalItems) {
    scan_local_kernel<T, Load, Store><<<1, kScanLocalBlock, 0, stream>>>(count, load, store);
    GS_LAUNCHED("scan_local_kernel");
    return GS_OK;
  }
  const int rounds = scan_rounds(count);
  const int64_t spans = scan_spans(count);
  GS_REQUIRE(spans <= 0x7fffffffLL, GS_ERR_OVERFLOW, "scan too large");
  scan_reduce_kernel<T, Load>
      <<<unsigned(spans), kScanBlock, 0, stream>>>(count, rounds, load, span_sums);
  GS_LAUNCHED("scan_reduce_kernel");
  scan_spans_kernel<T><<<1, kScanBlock, 0, stream>>>(span_sums, spans);
  GS_LAUNCHED("scan_spans_kernel");
  scan_down_kernel<T, Load, Store>
      <<<unsigned(spans), kScanBlock, 0, stream>>>(count, rounds, load, span_sums, store);
  GS_LAUNCHED("scan_down_kernel");
  return GS_OK;
}

}  // namespace gs
