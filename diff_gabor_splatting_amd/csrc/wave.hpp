// Wave64 cross-lane primitives for gfx950.
//
// wave_reduce_scatter<N> sums an N-value per-lane vector over the 64 lanes
// of a wavefront by recursive halving: at each of the six lane bits the
// vector is split in two halves, lanes with the bit clear keep the lower
// half and lanes with the bit set keep the upper half, and each lane adds
// its partner's copy of the half it keeps. After six steps lane L holds the
// complete wave sum of parameter rs_param<N>(L) (values >= N are padding).
// That costs about 2N cross-lane moves + adds instead of 6N for N separate
// butterfly reductions, and the final sums sit one per lane, so a single
// vector atomic (LDS or global) publishes all N of them.
//
// Bits 3..0 use DPP row_mirror, row_half_mirror and quad permutations, each
// of which pairs every lane with bit B clear with a lane that has bit B set
// inside the same group; bits 5 and 4 use the gfx950 v_permlane32_swap /
// v_permlane16_swap instructions (one instruction exchanges two halves).
// Any pairing that flips bit B and keeps the bits already reduced is all
// the reduction needs.
#pragma once

#include <hip/hip_runtime.h>

namespace gs {

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// DPP control codes (GFX9 encoding).
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]

template <int Ctrl>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_amdgcn_update_dpp(0.0f, v, Ctrl, 0xf, 0xf, false);
}

// Combine halves `lo` and `hi` across the lane pair split by bit B:
// lanes with bit B clear return lo + partner's lo, the others hi + partner's hi.
template <int B>
__device__ __forceinline__ float exchange_add(float lo, float hi, int lane) {
  if constexpr (B == 5) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false,
                                              false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else if constexpr (B == 4) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false,
                                              false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else if constexpr (B == 3 || B == 2) {
    // Mirror pairs never leave a bank pair: bit 3 splits every 16-lane row
    // into banks {0,1} | {2,3}, bit 2 into banks {0,2} | {1,3}. Two DPP adds,
    // each writing only the banks that keep its half, replace the per-lane
    // selects. The s_nop gives the two wait states a DPP source read needs
    // after a VALU write.
    float r;
    if constexpr (B == 3) {
      asm("s_nop 1\n\t"
          "v_add_f32_dpp %0, %2, %2 row_mirror row_mask:0xf bank_mask:0xc\n\t"
          "v_add_f32_dpp %0, %1, %1 row_mirror row_mask:0xf bank_mask:0x3"
          : "=&v"(r)
          : "v"(lo), "v"(hi));
    } else {
      asm("s_nop 1\n\t"
          "v_add_f32_dpp %0, %2, %2 row_half_mirror row_mask:0xf bank_mask:0xa\n\t"
          "v_add_f32_dpp %0, %1, %1 row_half_mirror row_mask:0xf bank_mask:0x5"
          : "=&v"(r)
          : "v"(lo), "v"(hi));
    }
    return r;
  } else {
    const bool upper = (lane >> B) & 1;
    const float send = upper ? lo : hi;
    const float keep = upper ? hi : lo;
    constexpr int ctrl = B == 3 ? kDppRowMirror
                         : B == 2 ? kDppRowHalfMirror
                         : B == 1 ? kDppQuadXor2
                                  : kDppQuadXor1;
    return keep + dpp_move<ctrl>(send);
  }
}

// Four bank-masked mirror exchanges (bits 3 or 2, see exchange_add) in one
// block: their inputs were all written before it, so one s_nop covers the
// DPP read hazard of all eight adds.
template <int B>
__device__ __forceinline__ void exchange_add4(const float* lo, const float* hi, float* out) {
  static_assert(B == 3 || B == 2, "bank-masked exchanges exist for lane bits 3 and 2");
  if constexpr (B == 3) {
    asm("s_nop 1\n\t"
        "v_add_f32_dpp %0, %8, %8 row_mirror row_mask:0xf bank_mask:0xc\n\t"
        "v_add_f32_dpp %0, %4, %4 row_mirror row_mask:0xf bank_mask:0x3\n\t"
        "v_add_f32_dpp %1, %9, %9 row_mirror row_mask:0xf bank_mask:0xc\n\t"
        "v_add_f32_dpp %1, %5, %5 row_mirror row_mask:0xf bank_mask:0x3\n\t"
        "v_add_f32_dpp %2, %10, %10 row_mirror row_mask:0xf bank_mask:0xc\n\t"
        "v_add_f32_dpp %2, %6, %6 row_mirror row_mask:0xf bank_mask:0x3\n\t"
        "v_add_f32_dpp %3, %11, %11 row_mirror row_mask:0xf bank_mask:0xc\n\t"
        "v_add_f32_dpp %3, %7, %7 row_mirror row_mask:0xf bank_mask:0x3"
        : "=&v"(out[0]), "=&v"(out[1]), "=&v"(out[2]), "=&v"(out[3])
        : "v"(lo[0]), "v"(lo[1]), "v"(lo[2]), "v"(lo[3]), "v"(hi[0]), "v"(hi[1]), "v"(hi[2]),
          "v"(hi[3]));
  } else {
    asm("s_nop 1\n\t"
        "v_add_f32_dpp %0, %8, %8 row_half_mirror row_mask:0xf bank_mask:0xa\n\t"
        "v_add_f32_dpp %0, %4, %4 row_half_mirror row_mask:0xf bank_mask:0x5\n\t"
        "v_add_f32_dpp %1, %9, %9 row_half_mirror row_mask:0xf bank_mask:0xa\n\t"
        "v_add_f32_dpp %1, %5, %5 row_half_mirror row_mask:0xf bank_mask:0x5\n\t"
        "v_add_f32_dpp %2, %10, %10 row_half_mirror row_mask:0xf bank_mask:0xa\n\t"
        "v_add_f32_dpp %2, %6, %6 row_half_mirror row_mask:0xf bank_mask:0x5\n\t"
        "v_add_f32_dpp %3, %11, %11 row_half_mirror row_mask:0xf bank_mask:0xa\n\t"
        "v_add_f32_dpp %3, %7, %7 row_half_mirror row_mask:0xf bank_mask:0x5"
        : "=&v"(out[0]), "=&v"(out[1]), "=&v"(out[2]), "=&v"(out[3])
        : "v"(lo[0]), "v"(lo[1]), "v"(lo[2]), "v"(lo[3]), "v"(hi[0]), "v"(hi[1]), "v"(hi[2]),
          "v"(hi[3]));
  }
}

template <int B, int N>
__device__ __forceinline__ void rs_step(const float* in, float* out, int lane) {
  constexpr int H = (N + 1) / 2;
  // Bank-masked exchanges go four to a block; the rest one at a time.
  constexpr int kGrouped = (B == 3 || B == 2) ? H / 4 * 4 : 0;
#pragma unroll
  for (int i = 0; i < kGrouped; i += 4) {
    float lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      lo[k] = in[i + k];
      hi[k] = (i + k + H < N) ? in[i + k + H] : 0.0f;
    }
    if constexpr (kGrouped > 0) exchange_add4<(B == 3 ? 3 : 2)>(lo, hi, out + i);
  }
#pragma unroll
  for (int i = kGrouped; i < H; ++i) {
    const float lo = in[i];
    const float hi = (i + H < N) ? in[i + H] : 0.0f;
    out[i] = exchange_add<B>(lo, hi, lane);
  }
}

// The lane bits are reduced in the order 3, 2, 1, 0, 5, 4: the first steps
// move the most values, so they take the cheapest exchange (two bank-masked
// DPP adds per pair), the quad steps with their per-lane selects follow,
// and the row-crossing permlane swaps, which cost more than a plain VALU
// instruction, come last, once the vector has shrunk to a few values. The
// swaps then read values written by compiler-visible instructions, whose
// hazards the compiler resolves (it does not see into inline assembly).
// Half sizes after each step of an N-value reduction:
template <int N>
struct RsShape {
  static constexpr int h3 = (N + 1) / 2;
  static constexpr int h2 = (h3 + 1) / 2;
  static constexpr int h1 = (h2 + 1) / 2;
  static constexpr int h0 = (h1 + 1) / 2;
  static constexpr int h5 = (h0 + 1) / 2;
  static constexpr int h4 = (h5 + 1) / 2;
};

// Parameter index whose total lane `lane` holds after wave_reduce_scatter<N>,
// or N for a lane left with padding. Every step splits the vector at its
// fixed half size (RsShape); the lane's share of real values, a prefix of
// its vector, is followed through the steps, and a lane whose share runs
// out holds padding (exactly zero).
template <int N>
__device__ __forceinline__ int rs_param(int lane) {
  using S = RsShape<N>;
  constexpr int kBits[6] = {3, 2, 1, 0, 5, 4};
  constexpr int kHalf[6] = {S::h3, S::h2, S::h1, S::h0, S::h5, S::h4};
  int first = 0, count = N;
#pragma unroll
  for (int step = 0; step < 6; ++step) {
    const int half = kHalf[step];
    if ((lane >> kBits[step]) & 1) {
      first += half;
      count = count > half ? count - half : 0;
    } else {
      count = count < half ? count : half;
    }
  }
  return count > 0 ? first : N;
}

// All 64 lanes must be active. Returns this lane's total (see rs_param).
template <int N>
__device__ __forceinline__ float wave_reduce_scatter(const float (&v)[N], int lane) {
  static_assert(N >= 1 && N <= 64, "one reduce-scatter covers at most 64 values");
  using S = RsShape<N>;
  float a[S::h3], b[S::h2], c[S::h1], d[S::h0], e[S::h5], f[S::h4];
  rs_step<3, N>(v, a, lane);
  rs_step<2, S::h3>(a, b, lane);
  rs_step<1, S::h2>(b, c, lane);
  rs_step<0, S::h1>(c, d, lane);
  rs_step<5, S::h0>(d, e, lane);
  rs_step<4, S::h5>(e, f, lane);
  return f[0];
}

// wave_reduce_quads<N>: the same sums, distributed per quad. Recursive
// halving runs over lane bits 3, 2, 5 and 4 only, which leaves each lane a
// slice of Q = RsQuadShape<N>::h4 (at most 4) partial sums shared by the
// four lanes of its quad (lane bits 1 and 0); a butterfly of two DPP adds
// per value then completes those sums in every lane of the quad. Lane
// `lane` holds the total of parameter rs_quad_param<N>(lane) in the value it
// returns (N for a lane whose quad position is past its slice). For N = 33
// that is 74 VALU operations instead of the 82 of wave_reduce_scatter,
// whose quad-level halving steps need two selects per value.
template <int N>
struct RsQuadShape {
  static constexpr int h3 = (N + 1) / 2;
  static constexpr int h2 = (h3 + 1) / 2;
  static constexpr int h5 = (h2 + 1) / 2;
  static constexpr int h4 = (h5 + 1) / 2;
};

template <int N>
__device__ __forceinline__ int rs_quad_param(int lane) {
  using S = RsQuadShape<N>;
  constexpr int kBits[4] = {3, 2, 5, 4};
  constexpr int kHalf[4] = {S::h3, S::h2, S::h5, S::h4};
  int first = 0, count = N;
#pragma unroll
  for (int step = 0; step < 4; ++step) {
    const int half = kHalf[step];
    if ((lane >> kBits[step]) & 1) {
      first += half;
      count = count > half ? count - half : 0;
    } else {
      count = count < half ? count : half;
    }
  }
  const int q = lane & 3;
  return q < count ? first + q : N;
}

// All 64 lanes must be active. Returns this lane's total (see rs_quad_param).
template <int N>
__device__ __forceinline__ float wave_reduce_quads(const float (&v)[N], int lane) {
  static_assert(N >= 1 && N <= 64, "one reduction covers at most 64 values");
  using S = RsQuadShape<N>;
  static_assert(S::h4 <= 4, "a quad publishes at most four values");
  float a[S::h3], b[S::h2], c[S::h5], d[S::h4];
  rs_step<3, N>(v, a, lane);
  rs_step<2, S::h3>(a, b, lane);
  rs_step<5, S::h2>(b, c, lane);
  rs_step<4, S::h5>(c, d, lane);
  // Butterfly within the quad: every lane ends with the quad's sums.
#pragma unroll
  for (int i = 0; i < S::h4; ++i) {
    d[i] += dpp_move<kDppQuadXor1>(d[i]);
    d[i] += dpp_move<kDppQuadXor2>(d[i]);
  }
  const int q = lane & 3;
  float out = d[0];
#pragma unroll
  for (int i = 1; i < S::h4; ++i) out = q == i ? d[i] : out;
  return out;
}

// Full-wave integer maximum (all lanes receive the result).
__device__ __forceinline__ int wave_max(int v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v = max(v, __shfl_xor(v, offset, 64));
  return v;
}

// Full-wave float sum (all lanes receive the result).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
  return v;
}

}  // namespace gs
