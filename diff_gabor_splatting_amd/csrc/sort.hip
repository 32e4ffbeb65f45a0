// Kernel 3: stable LSD radix sort of (uint32 or uint64 key, int32 value)
// pairs.
//
// Each pass sorts on a digit of up to 8 bits, or 9 for 32-bit keys where
// that saves a pass (Merrill & Grimshaw's reduce-then-scan
// formulation, without decoupled look-back, so no workgroup ever waits on
// another):
//   1. upsweep  - every 4096-key span (2048 for short sorts) builds a digit
//                 histogram in LDS and stores it digit-major:
//                 counts[digit * spans + span];
//   2. scan     - one workgroup per digit scans that digit's counts over
//                 the spans (and the downsweep adds the digit totals'
//                 prefix), which yields, for every (digit, span), the first
//                 output slot;
//   3. downsweep- every span ranks its keys stably (wave-level digit match
//                 via ballots, per-wave running counters in LDS), stages the
//                 locally sorted span in LDS and writes it out so that runs
//                 of equal digits land on consecutive addresses.
// Sorts of up to 8192 keys run every pass in one workgroup instead
// (local_sort_kernel). Only bits [begin_bit, end_bit) are sorted. gs_sort_pairs sorts the
// reference's 64-bit image|tile|depth keys; the depth-first binning
// pipeline (binning.hip) sorts 32-bit depth keys and then 32-bit tile ids
// or tile-block ids.
#include "sort.hpp"

#include <type_traits>

#include "scan.hpp"

namespace gs {
namespace {

constexpr int kSortBlock = 256;
constexpr int kSortWaves = kSortBlock / 64;
// Keys per thread: 16 (4096-key spans), or 8 for sorts of up to
// kShortSort keys, which then spread over twice as many workgroups - a
// 1M-key sort otherwise leaves a 256-CU device with one span per CU.
constexpr int64_t kShortSort = int64_t(1) << 22;
__host__ __device__ constexpr int span_keys(int items) { return kSortBlock * items; }
int sort_items(int64_t m) { return m <= kShortSort ? 8 : 16; }
constexpr int kDigitBits = 8;
constexpr int kBins = 1 << kDigitBits;
// Multi-workgroup passes of 32-bit keys may take digits of up to
// kWideDigitBits bits (kWideBins bins) when that saves a pass: the 9-bit
// block-id sort of a 1080p image (510 tile blocks) then takes one pass
// instead of two. (Digits of 11 bits, which would sort 32-bit depth keys in
// three passes, measured slower: 2048-bin histograms and scans per span
// cost more than the pass they save.) The digit-major counts are sized for
// kWideBins.
constexpr int kWideDigitBits = 9;
constexpr int kWideBins = 1 << kWideDigitBits;

// Lanes of the wave whose `digit` equals this lane's: one ballot per digit
// bit, intersected. Invalid lanes belong to no group.
__device__ __forceinline__ uint64_t digit_peers(uint32_t digit, bool valid, int bits) {
  uint64_t peers = __ballot(valid);
  for (int b = 0; b < bits; ++b) {
    const bool set = (digit >> b) & 1u;
    const uint64_t vote = __ballot(set);
    peers &= set ? vote : ~vote;
  }
  return peers;
}

// Digit histogram of one span, stored digit-major: counts[digit * spans +
// span]. Each wave counts into its own LDS row; per key group the lowest
// lane adds the group's size, so skewed digits cost no atomic conflicts.
// Sorts whose length is known only on the device pass it as `live`: the
// grid then covers the capacity m, and the workgroups of spans past the live
// length return at once in every pass (the scan reads only the live spans'
// counts).
__device__ __forceinline__ int64_t live_length(int64_t m, const int64_t* live) {
  return live ? min(m, max(*live, int64_t(0))) : m;
}

template <typename Key, int Items, int Bins>
__global__ __launch_bounds__(kSortBlock) void radix_upsweep_kernel(
    const Key* __restrict__ keys, int64_t capacity, const int64_t* __restrict__ live, int shift,
    int bits, uint32_t* __restrict__ counts, int64_t spans) {
  const int64_t m = live_length(capacity, live);
  constexpr int kSortItems = Items;
  constexpr int kSortSpan = span_keys(Items);
  constexpr int kWaveSpan = 64 * Items;
  if (int64_t(blockIdx.x) * kSortSpan >= m) return;  // past the live length
  __shared__ uint32_t hist[kSortWaves][Bins];
  const int lane = __lane_id(), wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < kSortWaves * Bins; i += kSortBlock) (&hist[0][0])[i] = 0;
  __syncthreads();
  const uint32_t mask = (1u << bits) - 1u;
  const int64_t wave_base = int64_t(blockIdx.x) * kSortSpan + int64_t(wave) * kWaveSpan;
  Key key[kSortItems];
#pragma unroll
  for (int it = 0; it < kSortItems; ++it) {
    const int64_t i = wave_base + int64_t(it) * 64 + lane;
    key[it] = i < m ? keys[i] : Key(0);
  }
  // One LDS atomic per key, without a return value, so that a lane's 16
  // updates do not wait on each other; when every valid lane of the wave
  // holds the same digit (common in the high digits of depth keys) a single
  // add replaces 64 colliding ones.
#pragma unroll
  for (int it = 0; it < kSortItems; ++it) {
    const bool valid = wave_base + int64_t(it) * 64 + lane < m;
    const uint32_t digit = uint32_t(key[it] >> shift) & mask;
    const uint64_t live = __ballot(valid);
    const uint32_t first = __builtin_amdgcn_readfirstlane(digit);
    if (__all(!valid || digit == first)) {
      if (lane == 0 && live) atomicAdd(&hist[wave][first], uint32_t(__popcll(live)));
    } else if (valid) {
      atomicAdd(&hist[wave][digit], 1u);
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < Bins; d += kSortBlock) {
    uint32_t total = 0;
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) total += hist[w][d];
    counts[int64_t(d) * spans + blockIdx.x] = total;
  }
}

// Pass 2: workgroup d turns row d of the digit-major counts (the digit's
// count in every span) into exclusive prefixes along the row and writes the
// row's total; the downsweep adds the exclusive prefix of the 256 row
// totals, the digit's first output slot. One launch of 256 workgroups,
// each scanning `spans` counts, replaces a three-launch scan of all
// 256 * spans counts.
__global__ __launch_bounds__(kSortBlock) void scan_rows_kernel(uint32_t* __restrict__ counts,
                                                               int64_t spans,
                                                               uint32_t* __restrict__ totals,
                                                               int64_t capacity,
                                                               const int64_t* __restrict__ live,
                                                               int span) {
  __shared__ uint32_t partial[2][kSortWaves];
  const int lane = __lane_id(), wave = threadIdx.x >> 6;
  uint32_t* row = counts + int64_t(blockIdx.x) * spans;
  // The spans holding keys (all of them without a live length).
  const int64_t used = min(spans, (live_length(capacity, live) + span - 1) / span);
  uint32_t carry = 0;
  int parity = 0;
  for (int64_t base = 0; base < used; base += kSortBlock, parity ^= 1) {
    const int64_t i = base + threadIdx.x;
    const uint32_t v = i < used ? row[i] : 0u;
    const uint32_t incl = wave_inclusive_scan(v);
    if (lane == 63) partial[parity][wave] = incl;
    __syncthreads();
    uint32_t before = carry;
    for (int w = 0; w < wave; ++w) before += partial[parity][w];
    if (i < used) row[i] = before + incl - v;
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) carry += partial[parity][w];
  }
  if (threadIdx.x == 0) totals[blockIdx.x] = carry;
}

// Exclusive prefix over the workgroup of Bins values, each thread holding
// Bins / kSortBlock consecutive ones in `v` (in place), via `partial`
// (kSortWaves entries of LDS).
template <int Bins>
__device__ __forceinline__ void block_exclusive_scan(uint32_t (&v)[Bins / kSortBlock],
                                                     uint32_t* partial) {
  constexpr int kPer = Bins / kSortBlock;
  const int lane = __lane_id(), wave = threadIdx.x >> 6;
  uint32_t sum = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) sum += v[j];
  const uint32_t inclusive = wave_inclusive_scan(sum);
  if (lane == 63) partial[wave] = inclusive;
  __syncthreads();
  uint32_t run = inclusive - sum;
  for (int w = 0; w < wave; ++w) run += partial[w];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const uint32_t x = v[j];
    v[j] = run;
    run += x;
  }
}

// Values: whether int32 values travel with the keys (a keys-only sort
// passes null value arrays). Bins: digits of up to log2(Bins) bits.
template <typename Key, int Items, bool Values, int Bins>
__global__ __launch_bounds__(kSortBlock) void radix_downsweep_kernel(
    const Key* __restrict__ keys_in, const int* __restrict__ values_in,
    Key* __restrict__ keys_out, int* __restrict__ values_out, int64_t capacity,
    const int64_t* __restrict__ live, int shift, int bits, const uint32_t* __restrict__ offsets,
    const uint32_t* __restrict__ totals, int64_t spans) {
  const int64_t m = live_length(capacity, live);
  constexpr int kSortItems = Items;
  constexpr int kSortSpan = span_keys(Items);
  constexpr int kWaveSpan = 64 * Items;
  constexpr int kPer = Bins / kSortBlock;  // digits per thread in the digit passes
  if (int64_t(blockIdx.x) * kSortSpan >= m) return;  // past the live length
  __shared__ uint32_t running[kSortWaves][Bins];  // per-wave digit counters
  __shared__ uint32_t local_start[Bins];          // first local slot per digit
  __shared__ uint32_t global_start[Bins];         // first output slot per digit
  __shared__ uint32_t partial[2][kSortWaves];
  __shared__ Key stage_keys[kSortSpan];
  __shared__ int stage_values[Values ? kSortSpan : 1];
  const int lane = __lane_id(), wave = threadIdx.x >> 6;
  const uint32_t mask = (1u << bits) - 1u;
  for (int i = threadIdx.x; i < kSortWaves * Bins; i += kSortBlock) (&running[0][0])[i] = 0;
  __syncthreads();
  const int64_t span = blockIdx.x;

  const int64_t wave_base = span * kSortSpan + int64_t(wave) * kWaveSpan;
  const uint64_t lanes_below = (uint64_t(1) << lane) - 1;
  Key key[kSortItems];
  int value[kSortItems];
  uint32_t rank[kSortItems];
#pragma unroll
  for (int it = 0; it < kSortItems; ++it) {
    const int64_t i = wave_base + int64_t(it) * 64 + lane;
    const bool valid = i < m;
    key[it] = valid ? keys_in[i] : Key(0);
    value[it] = Values && valid ? values_in[i] : 0;
  }
  // Rank = keys of the same digit earlier in this wave's span: the group
  // leader reserves the group's slots with an LDS atomic that returns the
  // previous count (the atomics of a lane are issued back to back, in item
  // order, so the counts stay in key order), then every lane reads its
  // leader's value.
  uint32_t before[kSortItems];
  int leader[kSortItems];
#pragma unroll
  for (int it = 0; it < kSortItems; ++it) {
    const bool valid = wave_base + int64_t(it) * 64 + lane < m;
    const uint32_t digit = uint32_t(key[it] >> shift) & mask;
    const uint64_t peers = digit_peers(digit, valid, bits);
    leader[it] = peers ? __builtin_ctzll(peers) : lane;
    rank[it] = uint32_t(__popcll(peers & lanes_below));
    before[it] = 0;
    if (valid && (peers & lanes_below) == 0)
      before[it] = atomicAdd(&running[wave][digit], uint32_t(__popcll(peers)));
  }
#pragma unroll
  for (int it = 0; it < kSortItems; ++it) rank[it] += uint32_t(__shfl(int(before[it]), leader[it]));
  __syncthreads();
  // Per digit (thread t takes digits [kPer t, kPer (t + 1))): exclusive
  // offsets of each wave inside the span, the span's digit totals and their
  // exclusive prefix (the digit's first local slot), and the exclusive
  // prefix of the whole sequence's digit totals plus the digit's prefix
  // over the earlier spans (its first output slot).
  const int d0 = threadIdx.x * kPer;
  uint32_t local[kPer], global[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int d = d0 + j;
    uint32_t run = 0;
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) {
      const uint32_t c = running[w][d];
      running[w][d] = run;
      run += c;
    }
    local[j] = run;
    global[j] = totals[d];
  }
  block_exclusive_scan<Bins>(local, partial[0]);
  block_exclusive_scan<Bins>(global, partial[1]);
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int d = d0 + j;
    local_start[d] = local[j];
    global_start[d] = global[j] + offsets[int64_t(d) * spans + span];
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < kSortItems; ++it) {
    const int64_t i = wave_base + int64_t(it) * 64 + lane;
    if (i < m) {
      const uint32_t digit = uint32_t(key[it] >> shift) & mask;
      const uint32_t slot = local_start[digit] + running[wave][digit] + rank[it];
      if (slot < uint32_t(kSortSpan)) {  // always true when ranking is consistent
        stage_keys[slot] = key[it];
        if constexpr (Values) stage_values[slot] = value[it];
      }
    }
  }
  __syncthreads();
  const int64_t span_base = span * kSortSpan;
  const int span_count = int(min<int64_t>(kSortSpan, m - span_base));
  for (int slot = threadIdx.x; slot < span_count; slot += kSortBlock) {
    const Key k = stage_keys[slot];
    const uint32_t digit = uint32_t(k >> shift) & mask;
    const int64_t dst = int64_t(global_start[digit]) + (slot - int64_t(local_start[digit]));
    if (dst >= 0 && dst < m) {  // always true when the histograms are consistent
      keys_out[dst] = k;
      if constexpr (Values) values_out[dst] = stage_values[slot];
    }
  }
}

// Sorts of up to kLocalSort keys run in one workgroup of kLocalBlock
// threads, every pass in one launch: each thread keeps kLocalItems keys in
// registers (key i of wave w is item (i - w 64 kLocalItems) / 64 of lane
// i mod 64, so a wave's keys are ranked in order, as in the downsweep), the
// per-wave digit counters give every key its slot, and between passes the
// keys are restaged through LDS; the last pass writes the output.
constexpr int kLocalBlock = 1024;
constexpr int kLocalWaves = kLocalBlock / 64;
constexpr int kLocalItems = 8;
constexpr int64_t kLocalSort = int64_t(kLocalBlock) * kLocalItems;

template <typename Key, bool Values>
__global__ __launch_bounds__(kLocalBlock) void local_sort_kernel(
    const Key* __restrict__ keys_in, const int* __restrict__ values_in,
    Key* __restrict__ keys_out, int* __restrict__ values_out, int64_t capacity,
    const int64_t* __restrict__ live, int begin_bit, int end_bit, int passes, int digit_bits) {
  const int m = int(live_length(capacity, live));
  __shared__ uint32_t running[kLocalWaves][kBins];  // per-wave digit counters
  __shared__ uint32_t digit_start[kBins];
  __shared__ uint32_t wave_totals[kBins / 64];
  __shared__ Key stage_keys[kLocalSort];
  __shared__ int stage_values[Values ? kLocalSort : 1];
  const int lane = __lane_id(), wave = threadIdx.x >> 6;
  const int wave_base = wave * 64 * kLocalItems;
  const uint64_t lanes_below = (uint64_t(1) << lane) - 1;
  Key key[kLocalItems];
  int value[kLocalItems];
#pragma unroll
  for (int it = 0; it < kLocalItems; ++it) {
    const int i = wave_base + it * 64 + lane;
    key[it] = i < m ? keys_in[i] : Key(0);
    value[it] = Values && i < m ? values_in[i] : 0;
  }
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = begin_bit + pass * digit_bits;
    const int bits = min(digit_bits, end_bit - shift);
    const uint32_t mask = (1u << bits) - 1u;
    for (int i = threadIdx.x; i < kLocalWaves * kBins; i += kLocalBlock)
      (&running[0][0])[i] = 0;
    __syncthreads();
    uint32_t rank[kLocalItems], before[kLocalItems];
    int leader[kLocalItems];
#pragma unroll
    for (int it = 0; it < kLocalItems; ++it) {
      const bool valid = wave_base + it * 64 + lane < m;
      const uint32_t digit = uint32_t(key[it] >> shift) & mask;
      const uint64_t peers = digit_peers(digit, valid, bits);
      leader[it] = peers ? __builtin_ctzll(peers) : lane;
      rank[it] = uint32_t(__popcll(peers & lanes_below));
      before[it] = 0;
      if (valid && (peers & lanes_below) == 0)
        before[it] = atomicAdd(&running[wave][digit], uint32_t(__popcll(peers)));
    }
#pragma unroll
    for (int it = 0; it < kLocalItems; ++it)
      rank[it] += uint32_t(__shfl(int(before[it]), leader[it]));
    __syncthreads();
    // Per digit: each wave's first slot among the digit's keys, the
    // digit's total, then the exclusive prefix over digits (waves 0-3).
    if (threadIdx.x < kBins) {
      const int d = threadIdx.x;
      uint32_t run = 0;
      for (int w = 0; w < kLocalWaves; ++w) {
        const uint32_t c = running[w][d];
        running[w][d] = run;
        run += c;
      }
      const uint32_t incl = wave_inclusive_scan(run);
      if (lane == 63) wave_totals[wave] = incl;
      digit_start[d] = incl - run;
    }
    __syncthreads();
    if (threadIdx.x < kBins) {
      uint32_t below = 0;
      for (int w = 0; w < wave; ++w) below += wave_totals[w];
      digit_start[threadIdx.x] += below;
    }
    __syncthreads();
    const bool last = pass == passes - 1;
#pragma unroll
    for (int it = 0; it < kLocalItems; ++it) {
      const int i = wave_base + it * 64 + lane;
      if (i < m) {
        const uint32_t digit = uint32_t(key[it] >> shift) & mask;
        const uint32_t slot = digit_start[digit] + running[wave][digit] + rank[it];
        if (slot < uint32_t(m)) {  // always true when ranking is consistent
          if (last) {
            keys_out[slot] = key[it];
            if constexpr (Values) values_out[slot] = value[it];
          } else {
            stage_keys[slot] = key[it];
            if constexpr (Values) stage_values[slot] = value[it];
          }
        }
      }
    }
    if (!last) {
      __syncthreads();
#pragma unroll
      for (int it = 0; it < kLocalItems; ++it) {
        const int i = wave_base + it * 64 + lane;
        key[it] = i < m ? stage_keys[i] : Key(0);
        value[it] = Values && i < m ? stage_values[i] : 0;
      }
    }
  }
}

template <typename Key>
__global__ __launch_bounds__(256) void copy_pairs_kernel(const Key* __restrict__ keys_in,
                                                         const int* __restrict__ values_in,
                                                         Key* __restrict__ keys_out,
                                                         int* __restrict__ values_out,
                                                         int64_t capacity,
                                                         const int64_t* __restrict__ live) {
  const int64_t m = live_length(capacity, live);
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < m) {
    keys_out[i] = keys_in[i];
    if (values_in) values_out[i] = values_in[i];
  }
}

struct SortWorkspace {
  uint32_t* counts;       // kWideBins * spans
  uint32_t* totals;       // kWideBins: each digit's count over the whole sequence
  void* keys_tmp;         // m keys
  int* values_tmp;        // m
  size_t bytes;
};

SortWorkspace layout(void* base, int64_t m, int key_bytes) {
  const int64_t spans = ceil_div(m, span_keys(sort_items(m)));
  const int64_t count_items = int64_t(kWideBins) * spans;
  SortWorkspace w;
  size_t offset = 0;
  char* p = static_cast<char*>(base);
  w.counts = reinterpret_cast<uint32_t*>(p + offset);
  offset = align_up(offset + size_t(count_items) * 4, 256);
  w.totals = reinterpret_cast<uint32_t*>(p + offset);
  offset = align_up(offset + size_t(kWideBins) * 4, 256);
  w.keys_tmp = p + offset;
  offset = align_up(offset + size_t(m) * size_t(key_bytes), 256);
  w.values_tmp = reinterpret_cast<int*>(p + offset);  // unused by keys-only sorts
  offset = align_up(offset + size_t(m) * 4, 256);
  w.bytes = offset;
  return w;
}

}  // namespace

size_t radix_sort_workspace_bytes(int64_t m, int key_bytes) {
  if (m < 0) m = 0;
  return layout(nullptr, m, key_bytes).bytes + 256;
}

template <typename Key>
int radix_sort(const Key* keys_in, Key* keys_out, const int* values_in, int* values_out,
               int64_t m, int begin_bit, int end_bit, void* workspace, hipStream_t s,
               const int64_t* live) {
  if (m == 0) return GS_OK;
  SortWorkspace w = layout(workspace, m, int(sizeof(Key)));
  const int items = sort_items(m);
  const int64_t spans = ceil_div(m, span_keys(items));
  const int bits_total = end_bit - begin_bit;
  int passes = int(ceil_div(bits_total, kDigitBits));
  // Spread the bits evenly over the passes (13 bits: 7 + 6, not 8 + 5):
  // fewer digits per pass means longer runs of equal digits per span and
  // fewer ballots per key.
  int digit_bits = passes ? int(ceil_div(bits_total, passes)) : 0;
  if (passes == 0) {
    copy_pairs_kernel<Key><<<unsigned(ceil_div(m, 256)), 256, 0, s>>>(
        keys_in, values_in, keys_out, values_out, m, live);
    GS_LAUNCHED("copy_pairs_kernel");
    return GS_OK;
  }
  if (m <= kLocalSort) {
    auto local = [&](auto kernel) {
      kernel<<<1, kLocalBlock, 0, s>>>(keys_in, values_in, keys_out, values_out, m, live,
                                       begin_bit, end_bit, passes, digit_bits);
    };
    if (values_in) local(local_sort_kernel<Key, true>);
    else local(local_sort_kernel<Key, false>);
    GS_LAUNCHED("local_sort_kernel");
    return GS_OK;
  }
  // Wider digits for 32-bit keys when they save a pass.
  if (sizeof(Key) == 4) {
    const int wide_passes = int(ceil_div(bits_total, kWideDigitBits));
    if (wide_passes < passes) {
      passes = wide_passes;
      digit_bits = int(ceil_div(bits_total, passes));
    }
  }
  const int bins = digit_bits <= kDigitBits ? kBins : kWideBins;
  // Ping-pong so that the last pass writes the caller's output.
  const Key* src_k = keys_in;
  const int* src_v = values_in;
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = begin_bit + pass * digit_bits;
    const int bits = min(digit_bits, end_bit - shift);
    const bool to_output = ((passes - 1 - pass) % 2) == 0;
    Key* dst_k = to_output ? keys_out : static_cast<Key*>(w.keys_tmp);
    int* dst_v = values_in ? (to_output ? values_out : w.values_tmp) : nullptr;
    auto upsweep = [&](auto items_tag, auto bins_tag) {
      constexpr int I = decltype(items_tag)::value, B = decltype(bins_tag)::value;
      radix_upsweep_kernel<Key, I, B><<<unsigned(spans), kSortBlock, 0, s>>>(
          src_k, m, live, shift, bits, w.counts, spans);
    };
    auto downsweep = [&](auto items_tag, auto bins_tag) {
      constexpr int I = decltype(items_tag)::value, B = decltype(bins_tag)::value;
      if (values_in)
        radix_downsweep_kernel<Key, I, true, B><<<unsigned(spans), kSortBlock, 0, s>>>(
            src_k, src_v, dst_k, dst_v, m, live, shift, bits, w.counts, w.totals, spans);
      else
        radix_downsweep_kernel<Key, I, false, B><<<unsigned(spans), kSortBlock, 0, s>>>(
            src_k, src_v, dst_k, dst_v, m, live, shift, bits, w.counts, w.totals, spans);
    };
    auto run = [&](auto bins_tag) {
      using Items8 = std::integral_constant<int, 8>;
      using Items16 = std::integral_constant<int, 16>;
      constexpr int B = decltype(bins_tag)::value;
      if (items == 8) upsweep(Items8{}, bins_tag);
      else upsweep(Items16{}, bins_tag);
      GS_LAUNCHED("radix_upsweep_kernel");
      scan_rows_kernel<<<B, kSortBlock, 0, s>>>(w.counts, spans, w.totals, m, live,
                                                span_keys(items));
      GS_LAUNCHED("scan_rows_kernel");
      if (items == 8) downsweep(Items8{}, bins_tag);
      else downsweep(Items16{}, bins_tag);
      GS_LAUNCHED("radix_downsweep_kernel");
      return GS_OK;
    };
    const int status = bins == kBins ? run(std::integral_constant<int, kBins>{})
                                     : run(std::integral_constant<int, kWideBins>{});
    if (status != GS_OK) return status;
    src_k = dst_k;
    src_v = dst_v;
  }
  return GS_OK;
}

template int radix_sort<uint32_t>(const uint32_t*, uint32_t*, const int*, int*, int64_t, int,
                                  int, void*, hipStream_t, const int64_t*);
template int radix_sort<uint64_t>(const uint64_t*, uint64_t*, const int*, int*, int64_t, int,
                                  int, void*, hipStream_t, const int64_t*);

}  // namespace gs

extern "C" {

size_t gs_sort_workspace_size(int64_t m) { return gs::radix_sort_workspace_bytes(m, 8); }

size_t gs_sort32_workspace_size(int64_t m) { return gs::radix_sort_workspace_bytes(m, 4); }

int gs_sort_pairs32(const uint32_t* keys_in, uint32_t* keys_out, const int32_t* values_in,
                    int32_t* values_out, int64_t m, int32_t begin_bit, int32_t end_bit,
                    void* workspace, size_t workspace_bytes, void* stream) {
  using namespace gs;
  clear_error();
  GS_REQUIRE(m >= 0 && m <= 0x7fffffffLL, GS_ERR_OVERFLOW, "sort size exceeds int32");
  GS_REQUIRE(0 <= begin_bit && begin_bit <= end_bit && end_bit <= 32, GS_ERR_ARGUMENT,
             "invalid bit range [%d, %d)", begin_bit, end_bit);
  if (m == 0) return GS_OK;
  GS_REQUIRE(keys_in && keys_out && !values_in == !values_out, GS_ERR_ARGUMENT,
             "null pointer passed to gs_sort_pairs32");
  GS_REQUIRE(keys_in != keys_out && (!values_in || values_in != values_out), GS_ERR_ARGUMENT,
             "sort outputs must not alias inputs");
  const size_t need = gs_sort32_workspace_size(m);
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE,
             "sort needs %zu workspace bytes, got %zu", need, workspace_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_SORT, s);
  return radix_sort<uint32_t>(keys_in, keys_out, values_in, values_out, m, begin_bit, end_bit,
                              workspace, s);
}

int gs_sort_pairs(const uint64_t* keys_in, uint64_t* keys_out, const int32_t* values_in,
                  int32_t* values_out, int64_t m, int32_t begin_bit, int32_t end_bit,
                  void* workspace, size_t workspace_bytes, void* stream) {
  using namespace gs;
  clear_error();
  GS_REQUIRE(m >= 0 && m <= 0x7fffffffLL, GS_ERR_OVERFLOW, "sort size exceeds int32");
  GS_REQUIRE(0 <= begin_bit && begin_bit <= end_bit && end_bit <= 64, GS_ERR_ARGUMENT,
             "invalid bit range [%d, %d)", begin_bit, end_bit);
  if (m == 0) return GS_OK;
  GS_REQUIRE(keys_in && keys_out && values_in && values_out, GS_ERR_ARGUMENT,
             "null pointer passed to gs_sort_pairs");
  GS_REQUIRE(keys_in != keys_out && values_in != values_out, GS_ERR_ARGUMENT,
             "sort outputs must not alias inputs");
  const size_t need = gs_sort_workspace_size(m);
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE,
             "sort needs %zu workspace bytes, got %zu", need, workspace_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_SORT, s);
  return radix_sort<uint64_t>(keys_in, keys_out, values_in, values_out, m, begin_bit, end_bit,
                              workspace, s);
}

}  // extern "C"
