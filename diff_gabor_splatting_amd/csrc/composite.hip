// Kernels 4 and 5: forward and reverse tile compositors.
//
// Semantics follow the reference compositor (src/gabor_splatting/csrc/
// rasterize.cu:71-399):
//  * per (pixel, record): ray/plane intersection k = x T2 - T0,
//    l = y T2 - T1, p = k x l, (u, v) = p.xy / p.z; upstream low-pass filter
//    rho = min(u^2 + v^2, 2 |xy - pixel|^2); alpha = min(0.99, o exp(-rho/2));
//    records with alpha < 1/255, p.z == 0 or depth < near are skipped;
//  * front-to-back compositing that stops *before* a contribution that
//    would take transmittance below 1e-4, accumulating rgb, depth, normals
//    and the two-moment distortion, then adding T * background;
//  * backward replays each tile in reverse from its largest contributor
//    count, recovering T by division.
//
// MI355X design. Both kernels are bound by VALU issue (rocprof: ~95% of one
// wave64 VALU instruction per CU per cycle), so the work per (pixel,
// record) sample is what matters:
//  * one workgroup of four wave64s per 16x16 tile, each wave owning an 8x8
//    quadrant; records are staged in LDS in batches of 64 and read as
//    broadcasts;
//  * while staging, one thread per record derives per-record constants once
//    for all 256 pixels: a conservative rejection threshold on rho (2 ln(255
//    o), slightly enlarged) so most rejected samples cost ~25 instructions
//    and no division or exp; the four Gabor phases in revolutions,
//    t_f = A_f u + B_f v + C_f with A_f, B_f = m_f d_f and C_f = phase/2pi,
//    evaluated with the hardware sin/cos on fract(t_f); the colour mix
//    folded to W/2 (c1 + c2) + S (c1 - c2) with S = sum w_f/2 cos; the SIREN
//    pre-activations folded to zc + U u + V v;
//  * reciprocals (v_rcp) replace the IEEE divisions and exp2 replaces expf
//    (both within two float32 ulps);
//  * in the backward, each wave sums its 64 pixels' gradients with one
//    reduce-scatter (wave.hpp), adds them to a per-batch LDS accumulator with
//    one ds_add per wave, and after the batch the workgroup flushes nonzero
//    totals with one global atomic per (tile, record, parameter).
#include <climits>
#include <cmath>
#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "wave.hpp"

namespace gs {
namespace {

constexpr int kBatch = 64;

// Diagnostics build (-DGS_DIAGNOSTICS, libgabor_hip_diag.so): the
// compositors also stamp each tile's begin and end on the wall clock, the
// backward counts, per (record, wave) it processes, how many lanes take the
// record, and the forward counts the records its pixels visit. Targets are
// device pointers set by gs_diagnostics_set; a null target records nothing.
// The product build compiles none of this.
struct DiagnosticTargets {
  unsigned long long* lanes;  // [65]: processed (record, wave) pairs by taking lanes
  long long* forward_span;    // [tiles][2]: wall-clock begin, end of each tile
  long long* backward_span;   // [tiles][2]
  long long tiles;
  // [8] work counters (see gs_diagnostics_set): forward (pixel, record)
  // visits of in-image pixels, the forward's processed (record, wave) pairs
  // times 64 lanes; the backward's processed (record, wave) pairs and the
  // wave steps they would take with each 32-lane half (8x4) or each 16-lane
  // block (4x4) of the quadrant walking its own records: at best (per batch,
  // the largest count of any half or block) and in list order (records
  // taken by one half or block packed between those taken by several).
  unsigned long long* counters;
};

#ifdef GS_DIAGNOSTICS
// Step counts of one wave's batch in the backward under the half and block
// schedules above (scalar bookkeeping, identical in every lane).
struct PackingCounts {
  int any = 0, half[2] = {0, 0}, block[4] = {0, 0, 0, 0};
  int half_pending[2] = {0, 0}, block_pending[4] = {0, 0, 0, 0};
  int half_steps = 0, block_steps = 0;

  // One processed record with this ballot of taking lanes (lane = 8 y + x
  // over the 8x8 quadrant). Every array index is a compile-time constant, so
  // the counts stay in registers.
  __device__ __forceinline__ void add(uint64_t taking) {
    constexpr uint64_t kHalves[2] = {0x00000000FFFFFFFFull, 0xFFFFFFFF00000000ull};
    constexpr uint64_t kBlocks[4] = {0x000000000F0F0F0Full, 0x00000000F0F0F0F0ull,
                                     0x0F0F0F0F00000000ull, 0xF0F0F0F000000000ull};
    ++any;
    bool in_half[2], in_block[4];
    int halves = 0, blocks = 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      in_half[i] = (taking & kHalves[i]) != 0;
      half[i] += in_half[i];
      halves += in_half[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      in_block[i] = (taking & kBlocks[i]) != 0;
      block[i] += in_block[i];
      blocks += in_block[i];
    }
    if (halves == 1) {
#pragma unroll
      for (int i = 0; i < 2; ++i) half_pending[i] += in_half[i];
    } else {
      half_steps += max(half_pending[0], half_pending[1]) + 1;
      half_pending[0] = half_pending[1] = 0;
    }
    if (blocks == 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) block_pending[i] += in_block[i];
    } else {
      block_steps += max(max(block_pending[0], block_pending[1]),
                         max(block_pending[2], block_pending[3])) + 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) block_pending[i] = 0;
    }
  }

  // Adds the batch's counts to the workgroup's LDS counters [5] (lane 0)
  // and starts afresh.
  __device__ void flush(unsigned int* sums) {
    half_steps += max(half_pending[0], half_pending[1]);
    block_steps += max(max(block_pending[0], block_pending[1]),
                       max(block_pending[2], block_pending[3]));
    if (lane_id() == 0 && any) {
      atomicAdd(sums + 0, unsigned(any));
      atomicAdd(sums + 1, unsigned(max(half[0], half[1])));
      atomicAdd(sums + 2, unsigned(max(max(block[0], block[1]), max(block[2], block[3]))));
      atomicAdd(sums + 3, unsigned(half_steps));
      atomicAdd(sums + 4, unsigned(block_steps));
    }
    *this = PackingCounts();
  }
};
#endif
#ifdef GS_DIAGNOSTICS
__device__ DiagnosticTargets gs_diagnostics;

// A tile's span covers every workgroup that worked on it (the segments of a
// split tile): the earliest begin and the latest end. The caller sets
// begins to all ones and ends to zero.
__device__ __forceinline__ void stamp_tile(long long* span, int tile, long long begin) {
  if (threadIdx.x == 0 && span && tile < gs_diagnostics.tiles) {
    auto* stamps = reinterpret_cast<unsigned long long*>(span + 2 * int64_t(tile));
    atomicMin(stamps, static_cast<unsigned long long>(begin));
    atomicMax(stamps + 1, static_cast<unsigned long long>(wall_clock64()));
  }
}
#endif
constexpr float kTwoPi = 6.28318530717958647692f;
constexpr float kInvTwoPi = 0.15915494309189533577f;
constexpr float kNegHalfLog2e = -0.72134752044448170368f;  // -log2(e) / 2
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kSirenRevolutions = 30.f * kInvTwoPi;        // sin(30 z) = sin(2 pi z 30/2pi)
constexpr float kMinAlpha = 1.0f / 255.0f;

// Directions (cos(pi f / 4), sin(pi f / 4)) of the four Gabor frequencies,
// evaluated the way the reference does: float angle pi*f/4, float cos/sin.
__device__ constexpr float kDirX[4] = {1.0f, 0.70710677f, -4.371139e-08f, -0.70710677f};
__device__ constexpr float kDirY[4] = {0.0f, 0.70710677f, 1.0f, 0.70710677f};

__device__ __forceinline__ float rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float sin_rev(float t) { return __builtin_amdgcn_sinf(t); }
__device__ __forceinline__ float cos_rev(float t) { return __builtin_amdgcn_cosf(t); }
__device__ __forceinline__ float fract(float t) { return __builtin_amdgcn_fractf(t); }

// LDS row layouts (floats). Geometry first in both: T 0-8, xy 9-10,
// normal 11-13.
// The colour is HALF_W SUM_c + S DIFF_c: the forward's rows hold the
// product HALF_W SUM_c in the SUM slots (the forward needs no other use of
// SUM_c), the backward's rows hold SUM_c and HALF_W for the flush and the
// product at SUMW.
// THR (reject_threshold of the opacity) is written only for the full-list
// backward, the one reader of it (sample_surface with Reject); the replay
// backward keeps the record's list position in that slot instead (POS), so
// that it arrives with the row's other constants rather than in a separate
// dependent load.
struct ClassicRow {
  static constexpr int OP = 14, THR = 15;
  static constexpr int A = 16, B = 20, C = 24, HW = 28;  // 4 each
  static constexpr int HALF_W = 32, SUM = 33, DIFF = 36;  // 1, 3, 3
  static constexpr int POS = THR;  // replay backward: the record's list position (int bits)
  static constexpr int AP = 40, BP = 44;  // -2 pi HW_f A_f, -2 pi HW_f B_f (backward)
  static constexpr int SUMW = 48;         // HALF_W SUM_c (backward)
  static constexpr int STRIDE = 52;
  static constexpr int FORWARD_STRIDE = 40;  // the forward's rows end before AP
};
struct NeuralRow {
  static constexpr int OP = 14, THR = 15;
  static constexpr int POS = THR;  // replay backward: the record's list position (int bits)
  static constexpr int ZC = 16, U = 22, V = 28;  // 6 each
  static constexpr int W2 = 34, B2 = 52;         // 18, 3
  static constexpr int DIR = 55;                 // 3 (backward)
  static constexpr int WDIR = 58;                // W1[h][2..4], 18 (backward)
  static constexpr int STRIDE = 76;
  static constexpr int FORWARD_STRIDE = 60;  // the forward's rows: up to DIR, 16-byte aligned, rows 4 banks apart
};
// The neural forward's raw staging row: direction, then the appearance
// row's input weights and biases (appearance columns 0..35 at 3..38).
struct NeuralRaw {
  static constexpr int DIR = 0, W1 = 3, B1 = 33;
  static constexpr int WIDTH = 39;
};

// Forward: the forward compositor's rows, which leave out what only the
// adjoint reads (classic AP/BP, neural DIR/WDIR), so that six classic or
// four neural workgroups fit a CU's LDS.
template <bool Neural, bool Forward = false>
struct Layout {
  static constexpr int A = Neural ? kNeural : kClassic;  // raw appearance floats
  static constexpr int RAW = kGeometry + 1 + A;          // raw staging floats
  // The neural forward stages only what its row derivation reads (direction
  // 3, input weights 30, input biases 6: NeuralRaw); the gather writes the
  // rest straight into the rows.
  static constexpr int RAW_STRIDE = Neural ? (Forward ? 39 : 76) : 36;
  static constexpr int STRIDE = Neural ? (Forward ? NeuralRow::FORWARD_STRIDE : NeuralRow::STRIDE)
                                       : (Forward ? ClassicRow::FORWARD_STRIDE : ClassicRow::STRIDE);
  // Gradient values reduced per record: geometry columns 0..13, appearance
  // sums, opacity. The direction columns' gradients (classic: none) and the
  // neural input weights' direction columns are per-record constants times
  // the input-bias sums, applied at the flush, so they are not reduced:
  // neural appearance sums are input weights' columns 0, 1 (12), input
  // biases (6), output weights (18), output biases (3).
  static constexpr int NG = 14;
  static constexpr int AR = Neural ? 39 : A;
  static constexpr int NP = NG + AR + 1;
};
static_assert(Layout<true, true>::RAW_STRIDE == NeuralRaw::WIDTH,
              "the neural forward stages NeuralRaw rows");

// Offsets of the neural appearance sums (after the NG geometry values).
struct NeuralSums {
  static constexpr int W01 = 0, B1 = 12, W2 = 18, B2 = 36;
};

// Where the backward writes a record's appearance gradient: rows [P, A]
// (data[0]), or, with `columns`, for the neural renderer, the SIREN's four
// parameter groups as separate arrays (data[g] [P, width g]): input weights
// (appearance columns 0..29), input biases (30..35), output weights
// (36..53), output biases (54..56).
struct AppearanceGradient {
  float* data[4];
  bool columns;
};

// Float atomic add at a global-memory address held as an integer (a global
// atomic, as atomicAdd gives for a kernel argument's pointer, rather than the
// flat one a pointer of unknown address space would take).
__device__ __forceinline__ void global_add(uint64_t address, float value) {
  using GlobalFloat = __attribute__((address_space(1))) float;
  __hip_atomic_fetch_add((GlobalFloat*)address, value, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
}

// The address of neural appearance column `col` of primitive `prim` in the
// column-group layout.
__device__ __forceinline__ float* siren_column(const AppearanceGradient& g, int64_t prim,
                                               int col) {
  return col < 30   ? g.data[0] + prim * 30 + col
         : col < 36 ? g.data[1] + prim * 6 + (col - 30)
         : col < 54 ? g.data[2] + prim * 18 + (col - 36)
                    : g.data[3] + prim * 3 + (col - 54);
}

// Rejection threshold on rho: alpha = min(0.99, o exp(-rho/2)) < 1/255
// whenever rho > 2 ln(255 o). The relative and absolute slack keep the test
// conservative against float32 rounding, so it only ever skips samples the
// exact test rejects.
__device__ __forceinline__ float reject_threshold(float opacity) {
  return 2.f * logf(255.f * opacity) * (1.f + 1e-4f) + 1e-4f;
}

// Screen footprint of a record: the region where sample_surface can pass
// its footprint test, rho2 <= thr or rho3 <= thr.
//  * rho2 = 2 |xy - pixel|^2 <= thr is a disc of radius sqrt(thr / 2);
//  * rho3 = u^2 + v^2 of the ray's hit on the surface plane (u, v in the
//    plane's scaled axes, columns of T) is <= thr on the image of the disc
//    u^2 + v^2 <= thr. With the whole disc in front of the camera
//    (T22 > sqrt(thr) |(T20, T21)|) that image is an ellipse whose centre
//    and box follow from the dual conic C = T diag(thr, thr, -1) T^T: centre
//    C02 / C22 and half width sqrt(C02^2 - C00 C22) / |C22| (y alike).
//    The numerator is expanded into 2x2 minors of rows 0 and 2 of T,
//    C02^2 - C00 C22 = thr (m02^2 + m12^2) - thr^2 m01^2, which avoids the
//    cancellation of two squared pixel coordinates. Otherwise the image is
//    unbounded.
//  * Inside the box, the ellipse is {Q <= 0} with Q = p0^2 + p1^2 - thr p2^2
//    and p = x a + y b + c, the affine function sample_surface evaluates as
//    k x l (a = t1 x t2, b = t2 x t0, c = t0 x t1 for the rows t of T).
// The box (x0, x1, y0, y1) bounds the union with a margin of 2% of the half
// extent plus one pixel, which keeps float rounding in here and in
// sample_surface from excluding an accepted pixel. Non-finite values give an
// unbounded box, thr <= 0 (no pixel can reach alpha >= 1/255) an empty one.
//
// record_reach derives these per-record constants once per batch into an
// LDS row of kReachPitch floats; quadrant_reach tests them against one wave's
// 8x8 quadrant.
struct ReachRow {
  static constexpr int BOX = 0;        // x0, x1, y0, y1
  static constexpr int CX = 4, CY = 5;  // ellipse centre
  static constexpr int A = 6, B = 9, C = 12;  // p = x a + y b + c
  static constexpr int QAA = 15, QBB = 16;    // Q's x^2 and y^2 coefficients
  static constexpr int THR = 17, X = 18, Y = 19;
  static constexpr int BOUNDED = 20;  // 1: test the ellipse exactly; 0: the box decides
};
constexpr int kReachPitch = 21;

__device__ void record_reach(const float* g, float thr, float* out) {
  constexpr float kHuge = 1e30f;
  using R = ReachRow;
  out[R::THR] = thr;
  out[R::X] = g[9];
  out[R::Y] = g[10];
  out[R::BOUNDED] = 0.f;
  if (!(thr > 0.f)) {
    out[R::BOX + 0] = kHuge;
    out[R::BOX + 1] = -kHuge;
    out[R::BOX + 2] = kHuge;
    out[R::BOX + 3] = -kHuge;
    return;
  }
  const float c = thr;
  const float disc = __builtin_amdgcn_sqrtf(0.5f * c);
  float x0 = g[9] - disc, x1 = g[9] + disc, y0 = g[10] - disc, y1 = g[10] + disc;
  float cx = 0.f, cy = 0.f;
  const float a = c * (g[6] * g[6] + g[7] * g[7]);
  const float c22 = a - g[8] * g[8];
  bool bounded = false;
  if (g[8] > 0.f && c22 < -1e-3f * (a + g[8] * g[8])) {
    const float inv = rcp(c22);
    // Row r of T against row 2: centre and half extent along that axis.
#pragma unroll
    for (int axis = 0; axis < 2; ++axis) {
      const float* t = g + 3 * axis;
      const float c02 = c * (t[0] * g[6] + t[1] * g[7]) - t[2] * g[8];
      const float m01 = t[0] * g[7] - t[1] * g[6];
      const float m02 = t[0] * g[8] - t[2] * g[6];
      const float m12 = t[1] * g[8] - t[2] * g[7];
      const float centre = c02 * inv;
      const float half =
          __builtin_amdgcn_sqrtf(fmaxf(c * (m02 * m02 + m12 * m12) - c * c * m01 * m01, 0.f)) *
          fabsf(inv);
      if (axis == 0) {
        cx = centre;
        x0 = fminf(x0, centre - half);
        x1 = fmaxf(x1, centre + half);
      } else {
        cy = centre;
        y0 = fminf(y0, centre - half);
        y1 = fmaxf(y1, centre + half);
      }
    }
    bounded = true;
  } else {
    x0 = y0 = -kHuge;  // the disc's image is unbounded: cull nothing
    x1 = y1 = kHuge;
  }
  const float mx = 1.f + 0.01f * (x1 - x0), my = 1.f + 0.01f * (y1 - y0);
  x0 -= mx;
  x1 += mx;
  y0 -= my;
  y1 += my;
  if (!(isfinite(x0) && isfinite(x1) && isfinite(y0) && isfinite(y1) && isfinite(cx) &&
        isfinite(cy))) {
    x0 = y0 = -kHuge;
    x1 = y1 = kHuge;
    bounded = false;
  }
  out[R::BOX + 0] = x0;
  out[R::BOX + 1] = x1;
  out[R::BOX + 2] = y0;
  out[R::BOX + 3] = y1;
  if (!bounded) return;
  const float* t0 = g;
  const float* t1 = g + 3;
  const float* t2 = g + 6;
  const float va[3] = {t1[1] * t2[2] - t1[2] * t2[1], t1[2] * t2[0] - t1[0] * t2[2],
                       t1[0] * t2[1] - t1[1] * t2[0]};
  const float vb[3] = {t2[1] * t0[2] - t2[2] * t0[1], t2[2] * t0[0] - t2[0] * t0[2],
                       t2[0] * t0[1] - t2[1] * t0[0]};
  const float vc[3] = {t0[1] * t1[2] - t0[2] * t1[1], t0[2] * t1[0] - t0[0] * t1[2],
                       t0[0] * t1[1] - t0[1] * t1[0]};
  const float qaa = va[0] * va[0] + va[1] * va[1] - thr * va[2] * va[2];
  const float qbb = vb[0] * vb[0] + vb[1] * vb[1] - thr * vb[2] * vb[2];
  if (!(qaa > 0.f && qbb > 0.f)) return;  // not elliptic after all: the box decides
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    out[R::A + k] = va[k];
    out[R::B + k] = vb[k];
    out[R::C + k] = vc[k];
  }
  out[R::CX] = cx;
  out[R::CY] = cy;
  out[R::QAA] = qaa;
  out[R::QBB] = qbb;
  out[R::BOUNDED] = 1.f;
}

// Whether any pixel of the 8x8 quadrant at (qx, qy) can pass the footprint
// test, decided on the rectangle R = [qx - 1/2, qx + 7 + 1/2] x (y alike):
//  * the box must meet the quadrant;
//  * the disc meets R when the point of R nearest its centre lies in it;
//  * Q is convex, so the ellipse meets R when its centre lies in R or when
//    the minimum of Q over an edge of R facing the centre is <= 0; along an
//    edge Q is a parabola, minimised at its clamped vertex.
// The half-pixel growth and a relative slack of 1e-3 on both comparisons
// keep float rounding from excluding a pixel the per-pixel test accepts.
__device__ bool quadrant_reach(const float* r, float qx, float qy) {
  using R = ReachRow;
  const bool in_box = (r[R::BOX + 1] >= qx) & (r[R::BOX + 0] <= qx + 7.f) &
                      (r[R::BOX + 3] >= qy) & (r[R::BOX + 2] <= qy + 7.f);
  if (!in_box) return false;
  if (r[R::BOUNDED] == 0.f) return true;
  constexpr float kGrow = 0.5f, kSlack = 1e-3f;
  const float thr = r[R::THR];
  const float x0 = qx - kGrow, x1 = qx + 7.f + kGrow;
  const float y0 = qy - kGrow, y1 = qy + 7.f + kGrow;
  const float dx = fminf(fmaxf(r[R::X], x0), x1) - r[R::X];
  const float dy = fminf(fmaxf(r[R::Y], y0), y1) - r[R::Y];
  if (2.f * (dx * dx + dy * dy) <= thr * (1.f + kSlack)) return true;
  const float cx = r[R::CX], cy = r[R::CY];
  const bool out_x = (cx < x0) | (cx > x1);
  const bool out_y = (cy < y0) | (cy > y1);
  if (!out_x && !out_y) return true;
  const float* a = r + R::A;
  const float* b = r + R::B;
  const float* c = r + R::C;
  bool hit = false;
  if (out_x) {  // edge x = ex, vertex of Q(ex, y) clamped to [y0, y1]
    const float ex = cx < x0 ? x0 : x1;
    const float u[3] = {ex * a[0] + c[0], ex * a[1] + c[1], ex * a[2] + c[2]};
    const float ub = u[0] * b[0] + u[1] * b[1] - thr * u[2] * b[2];
    const float y = fminf(fmaxf(-ub * rcp(r[R::QBB]), y0), y1);
    const float p[3] = {u[0] + y * b[0], u[1] + y * b[1], u[2] + y * b[2]};
    const float plane = p[0] * p[0] + p[1] * p[1], axial = thr * p[2] * p[2];
    hit = plane - axial <= kSlack * (plane + axial);
  }
  if (out_y) {  // edge y = ey, vertex of Q(x, ey) clamped to [x0, x1]
    const float ey = cy < y0 ? y0 : y1;
    const float u[3] = {ey * b[0] + c[0], ey * b[1] + c[1], ey * b[2] + c[2]};
    const float ua = u[0] * a[0] + u[1] * a[1] - thr * u[2] * a[2];
    const float x = fminf(fmaxf(-ua * rcp(r[R::QAA]), x0), x1);
    const float p[3] = {u[0] + x * a[0], u[1] + x * a[1], u[2] + x * a[2]};
    const float plane = p[0] * p[0] + p[1] * p[1], axial = thr * p[2] * p[2];
    hit = hit | (plane - axial <= kSlack * (plane + axial));
  }
  return hit;
}

// A value that is the same in every lane, moved to scalar registers so
// that loops and branches over it are scalar.
__device__ __forceinline__ uint64_t wave_uniform(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
  return (uint64_t(hi) << 32) | lo;
}

struct Sample {
  float k[3], l[3], p[3], s[2], inv_pz, depth, e, alpha;
  bool surface;
};

// Intersection of the pixel ray with the record's surface, the low-pass
// filter and alpha (rasterize.cu:71-103). Returns whether this lane
// accepts the sample; lanes with live = false never do. Written without
// early returns so that the wave's control flow stays scalar: after the
// cheap rejection test (no division, no exp) the whole wave leaves at once
// when no lane can accept.
// StandIns: lanes that do not accept leave with finite stand-ins (alpha, e,
// inv_pz and s zero, depth one, surface false), so that an adjoint run by
// every lane of the wave multiplies them only by zeros.
// Reject = false drops the early wave-wide exit and the cheap test with it,
// for callers that evaluate the sample anyway: the test only ever rejects
// samples whose alpha falls below 1/255 (reject_threshold), so the lanes
// that accept are the same either way, and the row's threshold is not read.
template <bool Neural, bool StandIns = false, bool Reject = true>
__device__ __forceinline__ bool sample_surface(const float* r, float x, float y,
                                               float near_plane, bool live, Sample& v) {
  constexpr int OP = Neural ? NeuralRow::OP : ClassicRow::OP;
  constexpr int THR = Neural ? NeuralRow::THR : ClassicRow::THR;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    v.k[i] = x * r[6 + i] - r[i];
    v.l[i] = y * r[6 + i] - r[3 + i];
  }
  v.p[0] = v.k[1] * v.l[2] - v.k[2] * v.l[1];
  v.p[1] = v.k[2] * v.l[0] - v.k[0] * v.l[2];
  v.p[2] = v.k[0] * v.l[1] - v.k[1] * v.l[0];
  const float dx = r[9] - x, dy = r[10] - y;
  const float rho2 = 2.f * (dx * dx + dy * dy);
  bool pass = live & (v.p[2] != 0.f);
  if constexpr (Reject) {
    // min(rho3, rho2) > thr without dividing: rho3 = |p.xy|^2 / p.z^2.
    const float thr = r[THR];
    const bool far =
        (rho2 > thr) & (v.p[0] * v.p[0] + v.p[1] * v.p[1] > thr * (v.p[2] * v.p[2]));
    pass = pass & !far;
    if (!__any(pass)) return false;
  }
  v.inv_pz = rcp(v.p[2]);
  v.s[0] = v.p[0] * v.inv_pz;
  v.s[1] = v.p[1] * v.inv_pz;
  const float rho3 = v.s[0] * v.s[0] + v.s[1] * v.s[1];
  v.surface = rho3 <= rho2;
  v.depth = (Neural || v.surface) ? fmaf(v.s[0], r[6], fmaf(v.s[1], r[7], r[8])) : r[8];
  v.e = __builtin_amdgcn_exp2f(fminf(rho3, rho2) * kNegHalfLog2e);
  v.alpha = fminf(0.99f, r[OP] * v.e);
  const bool ok = pass & (v.depth >= near_plane) & isfinite(v.depth) & (v.alpha >= kMinAlpha);
  if constexpr (StandIns) {
    v.alpha = ok ? v.alpha : 0.f;
    v.depth = ok ? v.depth : 1.f;
    v.e = ok ? v.e : 0.f;
    v.inv_pz = ok ? v.inv_pz : 0.f;
    v.s[0] = ok ? v.s[0] : 0.f;
    v.s[1] = ok ? v.s[1] : 0.f;
    v.surface = ok & v.surface;
  }
  return ok;
}

// Appearance at local coordinates s. Classic keeps the per-frequency
// cos/sin for the backward; neural keeps the hidden sin/cos.
struct Shade {
  float color[3];
  float c[6], sn[6];  // classic: cos/sin of the 4 waves; neural: cos/sin of 6 units
  float S;            // classic: sum_f (w_f / 2) cos_f
};

template <bool Neural, bool Backward>
__device__ __forceinline__ void shade(const float* r, const float* s, Shade& a) {
  if constexpr (Neural) {
    float hidden[6];
#pragma unroll
    for (int h = 0; h < 6; ++h) {
      const float z = r[NeuralRow::ZC + h] + r[NeuralRow::U + h] * s[0] + r[NeuralRow::V + h] * s[1];
      const float t = fract(z * kSirenRevolutions);
      hidden[h] = sin_rev(t);
      a.sn[h] = hidden[h];
      if constexpr (Backward) a.c[h] = cos_rev(t);
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      float z = r[NeuralRow::B2 + c];
#pragma unroll
      for (int h = 0; h < 6; ++h) z += r[NeuralRow::W2 + c * 6 + h] * hidden[h];
      a.color[c] = rcp(1.f + __builtin_amdgcn_exp2f(-z * kLog2e));
    }
  } else {
    float S = 0.f;
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      // Two fused multiply-adds (the phase offset enters the inner one).
      const float t = fract(
          fmaf(r[ClassicRow::A + f], s[0], fmaf(r[ClassicRow::B + f], s[1], r[ClassicRow::C + f])));
      a.c[f] = cos_rev(t);
      if constexpr (Backward) a.sn[f] = sin_rev(t);
      S += r[ClassicRow::HW + f] * a.c[f];
    }
    a.S = S;
#pragma unroll
    for (int c = 0; c < 3; ++c)
      a.color[c] = fmaf(S, r[ClassicRow::DIFF + c],
                        r[(Backward ? ClassicRow::SUMW : ClassicRow::SUM) + c]);
  }
}

// A replay entry's second word: the record's position in the tile's list in
// the low bits, the quadrant bits above them.
constexpr int kReplayPositionBits = 28;
constexpr int kReplayPositionMask = (1 << kReplayPositionBits) - 1;

// Which records a wave composites: kReachTest tests every record's footprint
// against the wave's quadrant; kReplayMask reads the quadrant bits of a
// replay entry (bit 28 + w: wave w's quadrant took the record in the
// forward), staged per record in `entries`.
enum Select { kReachTest, kReplayMask };

// Stage `count` records: thread t < count brings record t's point-list
// entry and primitive id (read one batch ahead by the caller, so that the
// two dependent loads overlap the previous batch); four threads per record
// then gather its raw fields into LDS, and one thread per record derives
// the row's constants.
template <bool Neural, Select Which = kReachTest, bool Forward = false>
__device__ __forceinline__ uint64_t load_batch(float* rows, float* raw, float* reach_rows,
                                               int* ids, int64_t* prims, float tile_x,
                                               float tile_y,
                                               int count, int id, int64_t prim,
                                               const float* geometry, const float* appearance,
                                               const float* opacities, int entry = 0,
                                               int* entries = nullptr) {
  using L = Layout<Neural, Forward>;
  const int t = threadIdx.x;
  if (t < count) {  // (id, prim): this thread's record, fetched by the caller ahead of time
    ids[t] = id;
    prims[t] = prim;
    if constexpr (Which == kReplayMask) entries[t] = entry;
  }
  __syncthreads();
  {
    // Four threads per record (record t / 4, quarter t % 4), each bringing a
    // fixed slice of the record's geometry row (17 floats), its appearance row
    // (pairs of floats when the row width is even and the array starts on an
    // 8-byte boundary, as every row then does) and, for the last quarter, its
    // opacity: no divisions, one base address per array, every load issued
    // before the first LDS write.
    constexpr int kParts = kTilePixels / kBatch;
    const int record = t / kParts, q = t % kParts;
    if (record < count) {
      float* dst = raw + record * L::RAW_STRIDE;
      // The neural forward's destinations: geometry columns 0..13 and the
      // opacity go to the row, the direction to NeuralRaw; appearance columns
      // 0..35 (input weights, biases) to NeuralRaw, 36..56 (output weights,
      // biases) to the row.
      constexpr bool kSplitRaw = Neural && Forward;
      static_assert(!kSplitRaw || L::A % 2 == 1, "the paired gather writes the full raw layout");
      constexpr int kGeo = (kGeometry + kParts - 1) / kParts;
      const float* g = geometry + int64_t(ids[record]) * kGeometry;
      const int64_t prim_j = prims[record];
      float gv[kGeo];
#pragma unroll
      for (int k = 0; k < kGeo; ++k) {
        const int f = q * kGeo + k;
        gv[k] = f < kGeometry ? g[f] : 0.f;
      }
      const float opacity = q == kParts - 1 ? opacities[prim_j] : 0.f;
      const float* a = appearance + prim_j * L::A;
      const bool pairs = L::A % 2 == 0 && (reinterpret_cast<uintptr_t>(appearance) & 7u) == 0;
      if (pairs) {
        constexpr int kPairs = L::A / 2, kPer = (kPairs + kParts - 1) / kParts;
        float2 av[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
          const int f = q * kPer + k;
          av[k] = f < kPairs ? reinterpret_cast<const float2*>(a)[f] : make_float2(0.f, 0.f);
        }
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
          const int f = q * kPer + k;
          if (f < kPairs) {
            dst[kGeometry + 1 + 2 * f] = av[k].x;
            dst[kGeometry + 2 + 2 * f] = av[k].y;
          }
        }
      } else {
        constexpr int kPer = (L::A + kParts - 1) / kParts;
        float av[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
          const int f = q * kPer + k;
          av[k] = f < L::A ? a[f] : 0.f;
        }
        if constexpr (kSplitRaw) {
          float* row = rows + record * L::STRIDE;
#pragma unroll
          for (int k = 0; k < kPer; ++k) {
            const int f = q * kPer + k;
            if (f < L::A)
              (f < 36 ? dst + NeuralRaw::W1 + f : row + NeuralRow::W2 + (f - 36))[0] = av[k];
          }
        } else {
#pragma unroll
          for (int k = 0; k < kPer; ++k) {
            const int f = q * kPer + k;
            if (f < L::A) dst[kGeometry + 1 + f] = av[k];
          }
        }
      }
      if constexpr (kSplitRaw) {
        float* row = rows + record * L::STRIDE;
#pragma unroll
        for (int k = 0; k < kGeo; ++k) {
          const int f = q * kGeo + k;
          if (f < kGeometry) (f < 14 ? row + f : dst + NeuralRaw::DIR + (f - 14))[0] = gv[k];
        }
        if (q == kParts - 1) row[NeuralRow::OP] = opacity;
      } else {
#pragma unroll
        for (int k = 0; k < kGeo; ++k) {
          const int f = q * kGeo + k;
          if (f < kGeometry) dst[f] = gv[k];
        }
        if (q == kParts - 1) dst[kGeometry] = opacity;
      }
    }
  }
  __syncthreads();
  // Wave 1 derives each record's footprint constants while wave 0 derives
  // the row constants; after the barrier every wave tests the records (one
  // per lane) against its own 8x8 quadrant of the tile.
  const int wave = t >> 6;
  const int j = t & 63;
  if (Which == kReachTest && wave == 1 && j < count) {
    if constexpr (Neural && Forward) {
      // The row already holds T, xy and the opacity; wave 0 writes only
      // later columns of it.
      const float* r = rows + j * L::STRIDE;
      record_reach(r, reject_threshold(r[NeuralRow::OP]), reach_rows + j * kReachPitch);
    } else {
      const float* g = raw + j * L::RAW_STRIDE;
      record_reach(g, reject_threshold(g[kGeometry]), reach_rows + j * kReachPitch);
    }
  }
  if constexpr (Neural && Forward) {
    if (t < count) {
      using R = NeuralRow;
      using W = NeuralRaw;
      const float* g = raw + t * L::RAW_STRIDE;
      float* r = rows + t * L::STRIDE;
#pragma unroll
      for (int h = 0; h < 6; ++h) {
        const float* w1 = g + W::W1 + h * 5;
        r[R::ZC + h] = g[W::B1 + h] + w1[2] * g[W::DIR + 0] + w1[3] * g[W::DIR + 1] +
                       w1[4] * g[W::DIR + 2];
        r[R::U + h] = w1[0] / 3.f;
        r[R::V + h] = w1[1] / 3.f;
      }
    }
  } else if (t < count) {
    // Only the full-list backward's samples test the row's threshold
    // (sample_surface with Reject).
    constexpr bool kRowThreshold = !Forward && Which == kReachTest;
    const float* g = raw + t * L::RAW_STRIDE;
    const float opacity = g[kGeometry];
    const float* a = g + kGeometry + 1;
    float* r = rows + t * L::STRIDE;
#pragma unroll
    for (int i = 0; i < 14; ++i) r[i] = g[i];
    if constexpr (Neural) {
      using R = NeuralRow;
#pragma unroll
      for (int i = 0; i < 3; ++i)
        if constexpr (!Forward) r[R::DIR + i] = g[14 + i];
      r[R::OP] = opacity;
      if constexpr (kRowThreshold) r[R::THR] = reject_threshold(opacity);
      if constexpr (Which == kReplayMask)
        r[R::POS] = __int_as_float(entries[t] & kReplayPositionMask);
#pragma unroll
      for (int h = 0; h < 6; ++h) {
        const float* w1 = a + h * 5;
        r[R::ZC + h] = a[30 + h] + w1[2] * g[14] + w1[3] * g[15] + w1[4] * g[16];
        r[R::U + h] = w1[0] / 3.f;
        r[R::V + h] = w1[1] / 3.f;
#pragma unroll
        for (int k = 0; k < 3; ++k)
          if constexpr (!Forward) r[R::WDIR + h * 3 + k] = w1[2 + k];
      }
#pragma unroll
      for (int i = 0; i < 18; ++i) r[R::W2 + i] = a[36 + i];
#pragma unroll
      for (int i = 0; i < 3; ++i) r[R::B2 + i] = a[54 + i];
    } else {
      using R = ClassicRow;
      if constexpr (Which == kReplayMask)
        r[R::POS] = __int_as_float(entries[t] & kReplayPositionMask);
      r[R::OP] = opacity;
      if constexpr (kRowThreshold) r[R::THR] = reject_threshold(opacity);
      float half_w = 0.f;
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        r[R::A + f] = a[10 + f] * kDirX[f];
        r[R::B + f] = a[10 + f] * kDirY[f];
        r[R::C + f] = a[14 + f] * kInvTwoPi;
        r[R::HW + f] = 0.5f * a[6 + f];
        if constexpr (!Forward) {
          r[R::AP + f] = -kTwoPi * (0.5f * a[6 + f]) * r[R::A + f];
          r[R::BP + f] = -kTwoPi * (0.5f * a[6 + f]) * r[R::B + f];
        }
        half_w += 0.5f * a[6 + f];
      }
      r[R::HALF_W] = half_w;
#pragma unroll
      for (int c = 0; c < 3; ++c) {
        const float sum = a[c] + a[3 + c];
        if constexpr (Forward) {
          r[R::SUM + c] = half_w * sum;
        } else {
          r[R::SUM + c] = sum;
          r[R::SUMW + c] = half_w * sum;
        }
        r[R::DIFF + c] = a[c] - a[3 + c];
      }
    }
  }
  __syncthreads();
  if constexpr (Which == kReplayMask) {
    // Bit j of the ballot says that this wave's quadrant took record j.
    return __ballot(j < count && ((uint32_t(entries[j]) >> (28 + wave)) & 1u));
  } else {
    // Bit j of the ballot says that record j may touch this wave's quadrant.
    const bool reach = j < count && quadrant_reach(reach_rows + j * kReachPitch,
                                                   tile_x + float(wave & 1) * 8.f,
                                                   tile_y + float(wave >> 1) * 8.f);
    return __ballot(reach);
  }
}

// Replay lists. The forward records, per tile, the list entries that at
// least one pixel took, in list order, as int2 {point-list entry (pair
// index), position in the tile's list | quadrant bits << 28}: bit 28 + w is
// set when a pixel of wave w's 8x8 quadrant took the record. Taken records
// are exactly the ones the backward replays (a pixel takes every accepted
// record up to its last contributor), so the backward walks this list
// instead of the tile's whole list and skips the footprint tests.

// Wave 0 appends the taken records of one batch (count records from list
// position first, their entry ids still staged in ids) to the tile's replay
// list, which holds n entries so far. Returns the new length.
__device__ __forceinline__ int append_replay(const uint64_t* wave_taken, const int* ids,
                                             int2* list, int n, int first, int count) {
  const int j = lane_id();
  uint32_t quads = 0;
#pragma unroll
  for (int w = 0; w < kTilePixels / 64; ++w)
    quads |= uint32_t((wave_taken[w] >> j) & 1u) << w;
  const bool keep = j < count && quads != 0u;
  const uint64_t kept = __ballot(keep);
  if (keep) {
    const int slot =
        n + int(__builtin_amdgcn_mbcnt_hi(uint32_t(kept >> 32),
                                          __builtin_amdgcn_mbcnt_lo(uint32_t(kept), 0u)));
    list[slot] = make_int2(ids[j], int(uint32_t(first + j) | (quads << kReplayPositionBits)));
  }
  return n + __popcll(kept);
}

// Split tiles. A tile whose point list is longer than `length` records (a
// multiple of kBatch) is replayed by the backward in segments, one
// workgroup each: segment k takes the replay entries the forward appended
// while walking list records [k length, (k + 1) length). For it the forward
// writes checkpoints c_1 .. c_K (K = ceil(list length / length)): c_j is the
// per-pixel prefix state after the first j length records (c_K: the final
// state before the background), with the replay-list length at that point.
// The backward of segment k starts from c_{k+1}: its transmittance, and the
// sum over the later records of w dL/dw, which is linear in the prefix sums,
// from c_K - c_{k+1} (the backward's running suffix at that point).
struct Segments {
  int length;    // records per segment; 0: no tile is split
  int tiles;
  int capacity;  // checkpoint slots
  float* state;  // [capacity][kCheckpointFloats][kTilePixels], one slot per checkpoint
  int* index;    // [tiles]: a split tile's first slot (-1: not split); then
                 // [capacity]: the replay-list length at each slot's checkpoint
  int2* work;    // [tiles + capacity]: the forward's (tile, segment) pairs,
                 // heaviest first, in the index buffer after an even offset
};

// Ints of the index buffer before the forward's work list (kept 8-byte
// aligned), and the buffer's whole length.
__host__ __device__ constexpr int64_t segment_work_offset(int64_t tiles, int64_t capacity) {
  return (tiles + capacity + 1) / 2 * 2;
}
__host__ __device__ constexpr int64_t segment_index_length(int64_t tiles, int64_t capacity) {
  return segment_work_offset(tiles, capacity) + 2 * (tiles + capacity);
}

// Floats per pixel of a checkpoint slot: a checkpoint is T, the rgb prefix
// (3), depth, normals (3), m1, m2; during the forward a slot first holds its
// segment's relative results (13 values, see renderForward).
constexpr int kCheckpointFloats = 13;

__device__ __forceinline__ int segment_count(int list_length, int length) {
  return (length > 0 && list_length > length) ? (list_length + length - 1) / length : 1;
}

struct TilePixel {
  int image, px, py;
  bool inside;
  int64_t pixel;
};

__device__ __forceinline__ TilePixel tile_pixel(int tile, int width, int height, int tw,
                                                int th) {
  TilePixel t;
  t.image = tile / (tw * th);
  const int local = tile - t.image * (tw * th);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  t.px = (local % tw) * kTile + (wave & 1) * 8 + (lane & 7);
  t.py = (local / tw) * kTile + (wave >> 1) * 8 + (lane >> 3);
  t.inside = t.px < width && t.py < height;
  t.pixel = (int64_t(t.image) * height + t.py) * width + t.px;
  return t;
}

// The nine map channels in five groups - rgb (channels 0-2), alpha (3),
// depth (4), normals (5-7), distortion (8) - each with its own base pointer
// and element strides: channel k of group g at pixel p is
// data[g][p * pixel_stride[g] + k * channel_stride[g]]. One [I,H,W,9]
// tensor, five separate tensors and strided gradient views all fit.
constexpr int kMapGroups = GS_MAP_GROUPS;
__host__ __device__ constexpr int map_group(int c) {
  return c < 3 ? 0 : c == 3 ? 1 : c == 4 ? 2 : c < 8 ? 3 : 4;
}
__host__ __device__ constexpr int map_group_first(int g) {
  return g == 0 ? 0 : g == 1 ? 3 : g == 2 ? 4 : g == 3 ? 5 : 8;
}

template <typename T>
struct MapGroups {
  T* data[kMapGroups];
  int64_t pixel_stride[kMapGroups];
  int64_t channel_stride[kMapGroups];

  __device__ __forceinline__ int64_t offset(int c, int64_t pixel) const {
    const int g = map_group(c);
    return pixel * pixel_stride[g] + int64_t(c - map_group_first(g)) * channel_stride[g];
  }
};

// Longest-first tile scheduling. Tiles are independent, so their dispatch
// order changes no result; issuing the most expensive tiles first keeps a
// heavy tile that would otherwise start late from setting the kernel's
// length. One workgroup buckets tiles by log2(cost) (256 buckets, 1/16
// octave) and writes the permutation heaviest bucket first.
constexpr int kOrderBlock = 1024;
constexpr int kOrderBuckets = 256;

__device__ __forceinline__ int cost_bucket(int cost) {
  if (cost <= 0) return 0;
  return min(kOrderBuckets - 1, int(__log2f(float(cost) + 1.f) * 16.f));
}

__device__ __forceinline__ int wave_inclusive_sum(int v) {
  const int lane = lane_id();
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int up = __shfl_up(v, d, 64);
    if (lane >= d) v += up;
  }
  return v;
}

// Heaviest-first bucket starts, run by the first wave of the block: next[b]
// = the number of items in buckets heavier than b, and *total (if given)
// the number of items. Each lane takes four consecutive buckets of the
// descending order and one wave scan combines them.
__device__ __forceinline__ void bucket_starts(const int* count, int* next, int* total) {
  static_assert(kOrderBuckets == 4 * 64, "four buckets per lane");
  const int lane = lane_id();
  const int top = kOrderBuckets - 1 - 4 * lane;  // this lane's buckets: top, top - 1, ...
  int c[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) c[j] = count[top - j];
  const int own = c[0] + c[1] + c[2] + c[3];
  int run = wave_inclusive_sum(own) - own;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    next[top - j] = run;
    run += c[j];
  }
  if (total && lane == 63) *total = run;
}

// Inclusive prefix sum of v over the kOrderBlock threads; *chunk receives
// the block's total. wave_totals holds kOrderBlock / 64 ints of LDS. The
// block is synchronised on return, so wave_totals may be reused at once.
__device__ __forceinline__ int block_inclusive_sum(int v, int* wave_totals, int* chunk) {
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int incl = wave_inclusive_sum(v);
  if (lane == 63) wave_totals[wave] = incl;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kOrderBlock / 64; ++w) {
    const int t = wave_totals[w];
    before += w < wave ? t : 0;
    all += t;
  }
  *chunk = all;
  __syncthreads();
  return before + incl;
}

// cost: per-tile cost, or null to use the tile's list length from ranges.
// With seg.length > 0 (the forward of split tiles) it also assigns each
// tile longer than seg.length its ceil(length / seg.length) checkpoint
// slots, in tile order, into seg.index[0 .. tiles) (-1: not split, or past
// the capacity, which the host sizes so that it is never reached).
__global__ __launch_bounds__(kOrderBlock) void tile_order_kernel(const int* __restrict__ cost,
                                                                 const int2* __restrict__ ranges,
                                                                 int tiles,
                                                                 int* __restrict__ order,
                                                                 Segments seg) {
  __shared__ int count[kOrderBuckets];
  __shared__ int next[kOrderBuckets];
  __shared__ int scan[kOrderBlock];
  if (seg.length > 0) {
    int carry = 0;
    for (int first = 0; first < tiles; first += kOrderBlock) {
      const int t = first + threadIdx.x;
      const int k = t < tiles ? segment_count(ranges[t].y - ranges[t].x, seg.length) : 1;
      const int slots = k > 1 ? k : 0;
      int chunk;
      const int base = carry + block_inclusive_sum(slots, scan, &chunk) - slots;
      if (t < tiles) seg.index[t] = (slots > 0 && base + slots <= seg.capacity) ? base : -1;
      carry += chunk;
    }
    // The forward's (tile, segment) work list, heaviest first by the list
    // records each walks; entries past the work count are (-1, 0).
    for (int b = threadIdx.x; b < kOrderBuckets; b += kOrderBlock) count[b] = 0;
    __syncthreads();
    auto pieces = [&](int t) {
      return seg.index[t] >= 0 ? segment_count(ranges[t].y - ranges[t].x, seg.length) : 1;
    };
    auto piece_cost = [&](int t, int k, int n) {
      const int length = ranges[t].y - ranges[t].x;
      return n == 1 ? length : min(seg.length, length - k * seg.length);
    };
    for (int t = threadIdx.x; t < tiles; t += kOrderBlock) {
      const int n = pieces(t);
      for (int k = 0; k < n; ++k) atomicAdd(&count[cost_bucket(piece_cost(t, k, n))], 1);
    }
    __syncthreads();
    if (threadIdx.x < 64) bucket_starts(count, next, &scan[0]);
    __syncthreads();
    const int total = scan[0];
    for (int t = threadIdx.x; t < tiles; t += kOrderBlock) {
      const int n = pieces(t);
      for (int k = 0; k < n; ++k)
        seg.work[atomicAdd(&next[cost_bucket(piece_cost(t, k, n))], 1)] = make_int2(t, k);
    }
    for (int i = total + threadIdx.x; i < tiles + seg.capacity; i += kOrderBlock)
      seg.work[i] = make_int2(-1, 0);
    __syncthreads();
    for (int b = threadIdx.x; b < kOrderBuckets; b += kOrderBlock) count[b] = 0;
    __syncthreads();
  }
  for (int b = threadIdx.x; b < kOrderBuckets; b += kOrderBlock) count[b] = 0;
  __syncthreads();
  for (int t = threadIdx.x; t < tiles; t += kOrderBlock) {
    const int c = cost ? cost[t] : ranges[t].y - ranges[t].x;
    atomicAdd(&count[cost_bucket(c)], 1);
  }
  __syncthreads();
  if (threadIdx.x < 64) bucket_starts(count, next, nullptr);
  __syncthreads();
  for (int t = threadIdx.x; t < tiles; t += kOrderBlock) {
    const int c = cost ? cost[t] : ranges[t].y - ranges[t].x;
    order[atomicAdd(&next[cost_bucket(c)], 1)] = t;
  }
}

// Forward cost estimate of each tile, for images with few tiles per
// workgroup slot of the GPU (2-4 rounds of workgroups), where the forward's
// length is set by the heaviest tiles and a heavy tile that starts late
// leaves most of the GPU idle behind it. The list length orders such tiles
// poorly when the lists are about equally long: a tile's cost is how far its
// pixels walk before the 1e-4 transmittance rule stops them. One wave per
// tile walks the tile's list for four probe pixels, the centres of its 8x8
// quadrants, 64 records at a time: lane j takes list position first + j,
// evaluates the record's alpha at each probe (the acceptance tests of
// sample_surface), and a wave prefix sum of log2(1 - alpha) locates the
// record that stops each probe. The cost is the longest of the four walks
// (the workgroup walks its batches until every wave's pixels are done). It
// only orders the tiles: no result depends on it.
constexpr int kProbeMaxTiles = 6144;  // 4 rounds of 256 CUs x 6 workgroups

template <bool Neural>
__global__ __launch_bounds__(256) void tile_probe_kernel(
    int tiles, int width, int height, int tw, int th, const float* __restrict__ geometry,
    const float* __restrict__ opacities, const int64_t* __restrict__ primitive_ids,
    const int* __restrict__ point_list, const int2* __restrict__ ranges, float near_plane,
    int* __restrict__ cost) {
  const int tile = int(blockIdx.x) * (256 / 64) + int(threadIdx.x >> 6);
  if (tile >= tiles) return;  // uniform over the wave
  const int lane = lane_id();
  const int local = tile % (tw * th);
  const int x0 = (local % tw) * kTile, y0 = (local / tw) * kTile;
  const int2 range = ranges[tile];
  const int length = range.y - range.x;
  constexpr float kLog2Stop = -13.287712379549449f;  // log2(1e-4)
  float log_t[4];
  int walked[4];
  bool live[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int px = x0 + (q & 1) * 8 + 4, py = y0 + (q >> 1) * 8 + 4;
    log_t[q] = 0.f;
    live[q] = px < width && py < height;
    walked[q] = live[q] ? length : 0;
  }
  for (int first = 0; first < length && (live[0] | live[1] | live[2] | live[3]);
       first += 64) {
    const int position = first + lane;
    float step[4] = {0.f, 0.f, 0.f, 0.f};
    if (position < length) {
      const int id = point_list[range.x + position];
      const float* g = geometry + int64_t(id) * kGeometry;
      float t[11];
#pragma unroll
      for (int i = 0; i < 11; ++i) t[i] = g[i];
      const float o = opacities[primitive_ids[id]];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float x = float(x0 + (q & 1) * 8 + 4), y = float(y0 + (q >> 1) * 8 + 4);
        float k[3], l[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          k[i] = x * t[6 + i] - t[i];
          l[i] = y * t[6 + i] - t[3 + i];
        }
        const float p0 = k[1] * l[2] - k[2] * l[1];
        const float p1 = k[2] * l[0] - k[0] * l[2];
        const float p2 = k[0] * l[1] - k[1] * l[0];
        const float inv = rcp(p2);
        const float s0 = p0 * inv, s1 = p1 * inv;
        const float rho3 = s0 * s0 + s1 * s1;
        const float dx = t[9] - x, dy = t[10] - y;
        const float rho2 = 2.f * (dx * dx + dy * dy);
        const float depth =
            (Neural || rho3 <= rho2) ? fmaf(s0, t[6], fmaf(s1, t[7], t[8])) : t[8];
        const float alpha = fminf(0.99f, o * __builtin_amdgcn_exp2f(fminf(rho3, rho2) *
                                                                      kNegHalfLog2e));
        const bool ok = (p2 != 0.f) & (depth >= near_plane) & isfinite(depth) &
                        (alpha >= kMinAlpha);
        step[q] = ok ? __builtin_amdgcn_logf(1.f - alpha) : 0.f;
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float prefix = step[q];  // inclusive prefix sum over the wave's lanes
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float up = __shfl_up(prefix, d, 64);
        if (lane >= d) prefix += up;
      }
      const uint64_t stops = __ballot(log_t[q] + prefix < kLog2Stop);
      if (live[q] && stops) {
        walked[q] = min(length, first + __builtin_ctzll(stops) + 1);
        live[q] = false;
      }
      log_t[q] += __shfl(prefix, 63, 64);
    }
  }
  if (lane == 0)
    cost[tile] = max(max(walked[0], walked[1]), max(walked[2], walked[3]));
}

// The backward's workgroups when tiles are split: every (tile, segment) with
// its replay entries as cost, heaviest first, into segments[0 .. tiles +
// seg.capacity); entries past the segment count are (-1, 0) and their
// workgroups exit at once.
__device__ __forceinline__ int segment_cost(const Segments& seg, const int* replay_counts,
                                            int tile, int k, int count) {
  if (count == 1) return replay_counts[tile];
  const int* n = seg.index + seg.tiles + seg.index[tile];
  return n[k] - (k ? n[k - 1] : 0);
}

__global__ __launch_bounds__(kOrderBlock) void segment_order_kernel(
    const int2* __restrict__ ranges, const int* __restrict__ replay_counts, int tiles,
    Segments seg, int2* __restrict__ segments) {
  __shared__ int count[kOrderBuckets];
  __shared__ int next[kOrderBuckets];
  __shared__ int total;
  for (int b = threadIdx.x; b < kOrderBuckets; b += kOrderBlock) count[b] = 0;
  __syncthreads();
  auto segments_of = [&](int t) {
    return seg.index[t] >= 0 ? segment_count(ranges[t].y - ranges[t].x, seg.length) : 1;
  };
  for (int t = threadIdx.x; t < tiles; t += kOrderBlock) {
    const int n = segments_of(t);
    for (int k = 0; k < n; ++k)
      atomicAdd(&count[cost_bucket(segment_cost(seg, replay_counts, t, k, n))], 1);
  }
  __syncthreads();
  if (threadIdx.x < 64) bucket_starts(count, next, &total);
  __syncthreads();
  for (int t = threadIdx.x; t < tiles; t += kOrderBlock) {
    const int n = segments_of(t);
    for (int k = 0; k < n; ++k) {
      const int bucket = cost_bucket(segment_cost(seg, replay_counts, t, k, n));
      segments[atomicAdd(&next[bucket], 1)] = make_int2(t, k);
    }
  }
  for (int i = total + threadIdx.x; i < tiles + seg.capacity; i += kOrderBlock)
    segments[i] = make_int2(-1, 0);
}

// Largest contributor count of each tile (where the backward starts).
__global__ __launch_bounds__(kTilePixels) void tile_last_kernel(int width, int height, int tw,
                                                                int th,
                                                                const int* __restrict__ contributors,
                                                                int* __restrict__ tile_last) {
  __shared__ int wave_max_last[kTilePixels / 64];
  const int tile = blockIdx.x;
  const int image = tile / (tw * th);
  const int local = tile - image * (tw * th);
  const int px = (local % tw) * kTile + (threadIdx.x & 15);
  const int py = (local / tw) * kTile + (threadIdx.x >> 4);
  const int last = (px < width && py < height)
                       ? contributors[(int64_t(image) * height + py) * width + px]
                       : 0;
  const int w = wave_max(last);
  if (lane_id() == 0) wave_max_last[threadIdx.x >> 6] = w;
  __syncthreads();
  if (threadIdx.x == 0)
    tile_last[tile] = max(max(wave_max_last[0], wave_max_last[1]),
                          max(wave_max_last[2], wave_max_last[3]));
}

// The two compositor kernels carry the reference's kernel names
// (renderForward / renderBackward, rasterize.cu:230, :284): tools that split
// a trace by those names, such as the reference benchmark's kernel profile,
// find them here too.
//
// Replay: also write the tile's replay list (replay + range start, see
// append_replay) and its length (replay_counts[tile]).
// Per-pixel state of a front-to-back walk: the map sums (before the
// background), transmittance, the two depth moments, the last list position
// taken (counted from 1) and whether the pixel is finished.
struct Walk {
  float out[kMaps];
  float T, m1, m2;
  int last;
  bool done;
#ifdef GS_DIAGNOSTICS
  int stop_at;      // list position after the record that stopped the pixel (0: none)
  int wave_steps;   // (record, wave) pairs this wave processed
#endif
};

__device__ __forceinline__ void begin_walk(Walk& w, bool inside) {
#pragma unroll
  for (int c = 0; c < kMaps; ++c) w.out[c] = 0.f;
  w.T = 1.f;
  w.m1 = w.m2 = 0.f;
  w.last = 0;
  w.done = !inside;
#ifdef GS_DIAGNOSTICS
  w.stop_at = 0;
  w.wave_steps = 0;
#endif
}

// The forward's LDS: a batch of staged rows and their ids.
template <bool Neural>
struct ForwardStage {
  float* rows;
  float* raw;
  float* reach_rows;
  int* ids;
  int64_t* prims;
  uint64_t* wave_taken;
};

// Composites list positions [first, end) (counted from the tile's range
// start) into every unfinished pixel, front to back, stopping a pixel before
// a contribution that would take its transmittance below 1e-4. With Replay,
// wave 0 appends the records some pixel took to `replay_block` (n entries so
// far, returned). A pixel starts from the state in `w`: a whole tile starts
// at T = 1; so does a segment of a split tile, whose walk is then relative
// to the transmittance in front of it (and its stops are sufficient, not
// exact: see mergeSegments).
template <bool Neural, bool Replay>
__device__ __forceinline__ int walk_list(const ForwardStage<Neural>& st, int range_x, int first,
                                         int end, const int* __restrict__ point_list,
                                         const int64_t* __restrict__ primitive_ids,
                                         const float* __restrict__ geometry,
                                         const float* __restrict__ appearance,
                                         const float* __restrict__ opacities, float x, float y,
                                         float tile_x, float tile_y, float near_plane,
                                         float mscale, float mnear, int2* replay_block,
                                         Walk& w) {
  using L = Layout<Neural, true>;
  const int wave = threadIdx.x >> 6;
  // Point-list entry and primitive id of record threadIdx.x of the next
  // batch, read ahead: the entry while this batch is gathered, the id while
  // its records are composited.
  int next_id = 0;
  int64_t next_prim = 0;
  if (int(threadIdx.x) < min(kBatch, end - first)) {
    next_id = point_list[range_x + first + threadIdx.x];
    next_prim = primitive_ids[next_id];
  }
  // Replay bookkeeping (wave 0): entries written so far, and the previous
  // batch, whose taken records are appended once every wave has finished it
  // (before the next batch overwrites its staged ids).
  int replay_n = 0, batch_first = 0, batch_count = 0;
  for (int start = first; start < end; start += kBatch) {
    if (__syncthreads_count(w.done) == kTilePixels) break;
    if (Replay && wave == 0)
      replay_n = append_replay(st.wave_taken, st.ids, replay_block, replay_n, batch_first,
                               batch_count);
    const int count = min(kBatch, end - start);
    const int id = next_id;
    const int64_t prim = next_prim;
    const bool ahead = int(threadIdx.x) < min(kBatch, end - start - kBatch);
    if (ahead) next_id = point_list[range_x + start + kBatch + threadIdx.x];
    const uint64_t reach = load_batch<Neural, kReachTest, true>(
        st.rows, st.raw, st.reach_rows, st.ids, st.prims, tile_x, tile_y, count, id, prim,
        geometry, appearance, opacities);
    if (ahead) next_prim = primitive_ids[next_id];
    batch_first = start;
    batch_count = count;
    // Only the records whose footprint meets this wave's quadrant, in list
    // order. The loop runs in lockstep across the wave: finished lanes are
    // masked through `done` rather than leaving the loop, so that every
    // branch below is on a wave-wide (scalar) condition.
    uint64_t todo = __all(w.done) ? 0 : wave_uniform(reach);
    uint64_t taken = 0;  // records that a lane of this wave took
    while (todo) {
      const int j = __builtin_ctzll(todo);
      todo &= todo - 1;
      const float* r = st.rows + j * L::STRIDE;
      Sample v;
      const bool ok = sample_surface<Neural, false, false>(r, x, y, near_plane, !w.done, v);
#ifdef GS_DIAGNOSTICS
      ++w.wave_steps;
#endif
      if (!__any(ok)) continue;
      const float next = w.T * (1.f - v.alpha);
      const bool stop = ok & (next < 0.0001f);
#ifdef GS_DIAGNOSTICS
      if (stop) w.stop_at = start + j + 1;
#endif
      // Without a stopping lane every lane that accepts takes the record, and
      // some lane accepts: only a stop needs the wave-wide tests.
      bool take = ok;
      if (__any(stop)) {
        w.done |= stop;
        if (__all(w.done)) break;
        take = ok & !stop;
        if (!__any(take)) continue;
      }
      taken |= uint64_t(1) << j;
      Shade a;
      shade<Neural, false>(r, v.s, a);
      if (take) {
        const float wt = w.T * v.alpha;
        const float m = mscale - mnear * rcp(v.depth);
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          w.out[c] += wt * a.color[c];
          w.out[5 + c] += wt * r[11 + c];
        }
        w.out[4] += wt * v.depth;
        w.out[8] += wt * (m * m * (1.f - w.T) + w.m2 - 2.f * m * w.m1);
        w.m1 += wt * m;
        w.m2 += wt * m * m;
        w.T = next;
        w.last = start + j + 1;
      }
    }
    if (Replay && lane_id() == 0) st.wave_taken[wave] = taken;
  }
  if constexpr (Replay) {
    __syncthreads();
    if (wave == 0)
      replay_n = append_replay(st.wave_taken, st.ids, replay_block, replay_n, batch_first,
                               batch_count);
  }
  return replay_n;
}

// A segment's slot while the forward runs (before mergeSegments turns it
// into the checkpoint): the relative walk's T', its map sums (rgb, depth,
// normals), sum w' m, sum w' m^2, its own distortion sum, the last position
// taken and whether the relative walk finished the pixel.
constexpr int kSegmentResults = 13;
static_assert(kCheckpointFloats >= kSegmentResults, "a slot holds a segment's results");

// Forward compositor: one workgroup per tile, or per segment of a split tile
// (seg.work lists the (tile, segment) pairs heaviest first; a segment writes
// its relative sums and its replay entries, at its own block of the tile's
// replay list, and mergeSegments completes the tile).
// Replay: also write the tile's replay list (replay + range start, see
// append_replay) and its length (replay_counts[tile]).
template <bool Neural, bool Replay, bool Split>
__global__ __launch_bounds__(kTilePixels, Neural ? (Split ? 4 : 5) : 6) void renderForward(
    int width, int height, int tw, int th, const float* __restrict__ geometry,
    const float* __restrict__ appearance, const float* __restrict__ opacities,
    const int64_t* __restrict__ primitive_ids, const float* __restrict__ backgrounds,
    const int* __restrict__ point_list, const int2* __restrict__ ranges,
    const int* __restrict__ order, float near_plane, float far_plane, MapGroups<float> maps,
    float* __restrict__ state, int* __restrict__ contributors, int2* __restrict__ replay,
    int* __restrict__ replay_counts, Segments seg) {
  using L = Layout<Neural, true>;
  __shared__ __align__(16) float rows[kBatch * L::STRIDE];
  __shared__ __align__(16) float raw[kBatch * L::RAW_STRIDE];
  __shared__ float reach_rows[kBatch * kReachPitch];
  __shared__ int ids[kBatch];
  __shared__ int64_t prims[kBatch];
  __shared__ uint64_t wave_taken[kTilePixels / 64];
  const ForwardStage<Neural> st{rows, raw, reach_rows, ids, prims, wave_taken};
  // (tile, segment) of this workgroup; past the work count: nothing.
  const int2 piece = Split ? seg.work[blockIdx.x] : make_int2(order[blockIdx.x], 0);
  if (piece.x < 0) return;
  const int tile = piece.x;
#ifdef GS_DIAGNOSTICS
  const long long diag_begin = wall_clock64();
#endif
  const TilePixel tp = tile_pixel(tile, width, height, tw, th);
  const float x = float(tp.px), y = float(tp.py);
  const int wave = threadIdx.x >> 6;
  const float tile_x = float(tp.px - (wave & 1) * 8 - (lane_id() & 7));
  const float tile_y = float(tp.py - (wave >> 1) * 8 - (lane_id() >> 3));
  const int2 range = ranges[tile];
  const float mscale = far_plane / (far_plane - near_plane);
  const float mnear = mscale * near_plane;
  const int base = Split ? seg.index[tile] : -1;
  int first = 0, end = range.y - range.x;
  if (base >= 0) {
    first = piece.y * seg.length;
    end = min(first + seg.length, end);
  }
  Walk w;
  begin_walk(w, tp.inside);
  const int replay_n = walk_list<Neural, Replay>(
      st, range.x, first, end, point_list, primitive_ids, geometry, appearance, opacities, x, y,
      tile_x, tile_y, near_plane, mscale, mnear, replay + range.x + first, w);
#ifdef GS_DIAGNOSTICS
  if (gs_diagnostics.counters) {
    // A split tile's segments count their relative walks. Summed per
    // workgroup in LDS, then one global atomic per counter and workgroup.
    __shared__ unsigned long long diag_walk[2];
    if (threadIdx.x < 2) diag_walk[threadIdx.x] = 0ull;
    __syncthreads();
    const int visited = tp.inside ? (w.stop_at > 0 ? w.stop_at : end) - first : 0;
    atomicAdd(&diag_walk[0], static_cast<unsigned long long>(visited));
    if (lane_id() == 0)
      atomicAdd(&diag_walk[1], 64ull * static_cast<unsigned long long>(w.wave_steps));
    __syncthreads();
    if (threadIdx.x < 2) atomicAdd(gs_diagnostics.counters + threadIdx.x, diag_walk[threadIdx.x]);
  }
#endif
  if (Split && base >= 0) {
    // A segment of a split tile: its relative results and replay count.
    float* c = seg.state + int64_t(base + piece.y) * (kCheckpointFloats * kTilePixels) +
               threadIdx.x;
    const float results[kSegmentResults] = {
        w.T,      w.out[0], w.out[1], w.out[2], w.out[4], w.out[5], w.out[6],
        w.out[7], w.m1,     w.m2,     w.out[8], __int_as_float(w.last),
        w.done ? 1.f : 0.f};
#pragma unroll
    for (int q = 0; q < kSegmentResults; ++q) c[q * kTilePixels] = results[q];
    if (threadIdx.x == 0) seg.index[seg.tiles + base + piece.y] = replay_n;
  } else {
    if (Replay && threadIdx.x == 0) replay_counts[tile] = replay_n;
    if (tp.inside) {
#pragma unroll
      for (int c = 0; c < 3; ++c) w.out[c] += w.T * backgrounds[tp.image * 3 + c];
      w.out[3] = 1.f - w.T;
#pragma unroll
      for (int c = 0; c < kMaps; ++c)
        maps.data[map_group(c)][maps.offset(c, tp.pixel)] = w.out[c];
      state[tp.pixel * 3 + 0] = w.T;
      state[tp.pixel * 3 + 1] = w.m1;
      state[tp.pixel * 3 + 2] = w.m2;
      contributors[tp.pixel] = w.last;
    }
  }
#ifdef GS_DIAGNOSTICS
  __syncthreads();
  stamp_tile(gs_diagnostics.forward_span, tile, diag_begin);
#endif
}

// Completes every split tile (one workgroup each; other tiles exit): walks
// its segments' results in list order per pixel, with the transmittance T
// in front of segment k. A segment whose relative walk did not finish the
// pixel and whose T' keeps T T' >= 1e-4 is merged in closed form:
//   sums += T sums', T *= T', m1 += T sum w'm, m2 += T sum w'm^2, and the
//   distortion gains T M2' + T^2 (dist' - M2') + T (m2 W' - 2 m1 M1')
//   (W' = 1 - T': its terms m^2 (1 - T T'_i) + m2 + T M2'_{<i} - 2 m (m1 +
//   T M1'_{<i}) expanded over the segment's records);
// otherwise the pixel stops inside segment k (a relative stop implies a
// stop: T T'(1 - alpha) <= T'(1 - alpha) < 1e-4), and the segment is walked
// again for the pixels concerned with their true transmittance, which
// applies the stop rule exactly. The records taken then are a subset of the
// relative walk's, whose replay entries therefore cover them. Writes the
// maps, state and contributors, checkpoint c_{k+1} into segment k's slot
// (the prefix state after it) and packs the segments' replay blocks into
// one list, with its running lengths as the checkpoints' replay lengths.
template <bool Neural>
__global__ __launch_bounds__(kTilePixels) void mergeSegments(
    int width, int height, int tw, int th, const float* __restrict__ geometry,
    const float* __restrict__ appearance, const float* __restrict__ opacities,
    const int64_t* __restrict__ primitive_ids, const float* __restrict__ backgrounds,
    const int* __restrict__ point_list, const int2* __restrict__ ranges, float near_plane,
    float far_plane, MapGroups<float> maps, float* __restrict__ state,
    int* __restrict__ contributors, int2* __restrict__ replay, int* __restrict__ replay_counts,
    Segments seg) {
  using L = Layout<Neural, true>;
  __shared__ __align__(16) float rows[kBatch * L::STRIDE];
  __shared__ __align__(16) float raw[kBatch * L::RAW_STRIDE];
  __shared__ float reach_rows[kBatch * kReachPitch];
  __shared__ int ids[kBatch];
  __shared__ int64_t prims[kBatch];
  __shared__ uint64_t wave_taken[kTilePixels / 64];
  const ForwardStage<Neural> st{rows, raw, reach_rows, ids, prims, wave_taken};
  const int tile = blockIdx.x;
  const int base = seg.index[tile];
  if (base < 0) return;
  const TilePixel tp = tile_pixel(tile, width, height, tw, th);
  const float x = float(tp.px), y = float(tp.py);
  const int wave = threadIdx.x >> 6;
  const float tile_x = float(tp.px - (wave & 1) * 8 - (lane_id() & 7));
  const float tile_y = float(tp.py - (wave >> 1) * 8 - (lane_id() >> 3));
  const int2 range = ranges[tile];
  const int length = range.y - range.x;
  const int pieces = segment_count(length, seg.length);
  const float mscale = far_plane / (far_plane - near_plane);
  const float mnear = mscale * near_plane;
  constexpr int kSlot = kCheckpointFloats * kTilePixels;
  Walk w;
  begin_walk(w, tp.inside);
  for (int k = 0; k < pieces; ++k) {
    float* c = seg.state + int64_t(base + k) * kSlot + threadIdx.x;
    float r[kSegmentResults];
#pragma unroll
    for (int q = 0; q < kSegmentResults; ++q) r[q] = c[q * kTilePixels];
    bool again = false;
    if (!w.done) {
      const float Tp = r[0];
      // (With 0.1% slack, so that a product rounded differently from the
      // record-by-record one never decides the stop.)
      if (r[12] != 0.f || w.T * Tp < 1.001e-4f) {
        again = true;
      } else {
        const float Ts = w.T;
        const float M1 = r[8], M2 = r[9];
        w.out[8] += Ts * M2 + Ts * Ts * (r[10] - M2) + Ts * (w.m2 * (1.f - Tp) - 2.f * w.m1 * M1);
        w.out[0] += Ts * r[1];
        w.out[1] += Ts * r[2];
        w.out[2] += Ts * r[3];
        w.out[4] += Ts * r[4];
        w.out[5] += Ts * r[5];
        w.out[6] += Ts * r[6];
        w.out[7] += Ts * r[7];
        w.m1 += Ts * M1;
        w.m2 += Ts * M2;
        w.T = Ts * Tp;
        const int last = __float_as_int(r[11]);
        if (last > 0) w.last = last;
      }
    }
    if (__syncthreads_or(again)) {
      // Exact walk of segment k for the pixels that stop inside it.
      const bool finished = w.done;
      w.done = finished || !again;
      const int first = k * seg.length;
      walk_list<Neural, false>(st, range.x, first, min(first + seg.length, length), point_list,
                               primitive_ids, geometry, appearance, opacities, x, y, tile_x,
                               tile_y, near_plane, mscale, mnear, nullptr, w);
      w.done = again ? w.done : finished;
    }
    // Checkpoint c_{k+1}: the prefix state after segment k (this thread's
    // column only, so no other thread's slot is touched).
    const float values[10] = {w.T,      w.out[0], w.out[1], w.out[2], w.out[4],
                              w.out[5], w.out[6], w.out[7], w.m1,     w.m2};
#pragma unroll
    for (int q = 0; q < 10; ++q) c[q * kTilePixels] = values[q];
  }
  // Pack the segments' replay blocks (segment k's entries start at list
  // position k * length) into one list. A block only moves left and never
  // onto a later block, and every chunk is read in full before it is
  // written, so no entry is overwritten before it is read.
  int* n = seg.index + seg.tiles + base;
  int packed = 0;
  for (int k = 0; replay && k < pieces; ++k) {
    const int count = n[k];
    __syncthreads();  // every thread has read n[k] before thread 0 rewrites it
    if (k > 0 && packed != k * seg.length) {
      const int2* src = replay + range.x + k * seg.length;
      int2* dst = replay + range.x + packed;
      for (int chunk = 0; chunk < count; chunk += kTilePixels) {
        const int i = chunk + int(threadIdx.x);
        const int2 e = i < count ? src[i] : make_int2(0, 0);
        __syncthreads();
        if (i < count) dst[i] = e;
      }
    }
    packed += count;
    if (threadIdx.x == 0) n[k] = packed;  // replay length at checkpoint c_{k+1}
  }
  if (replay && threadIdx.x == 0) replay_counts[tile] = packed;
  if (tp.inside) {
#pragma unroll
    for (int c = 0; c < 3; ++c) w.out[c] += w.T * backgrounds[tp.image * 3 + c];
    w.out[3] = 1.f - w.T;
#pragma unroll
    for (int c = 0; c < kMaps; ++c) maps.data[map_group(c)][maps.offset(c, tp.pixel)] = w.out[c];
    state[tp.pixel * 3 + 0] = w.T;
    state[tp.pixel * 3 + 1] = w.m1;
    state[tp.pixel * 3 + 2] = w.m2;
    contributors[tp.pixel] = w.last;
  }
}

// Appearance adjoint given dL/dcolor = gc. Writes the summands of the
// per-record appearance sums into ga (classic 18; neural 39, laid out as
// NeuralSums) and accumulates d/d(u, v) into gs. The neural input weights'
// direction columns and the direction itself receive gz_h d_k and
// gz_h W1[h][2 + k]: per-record constants times the input-bias summand gz_h,
// applied once per record at the flush (neural_outputs).
template <bool Neural>
__device__ __forceinline__ void shade_backward(const float* r, const float* s, const Shade& a,
                                               const float* gc, float* ga, float* gs) {
  if constexpr (Neural) {
    using R = NeuralRow;
    using S = NeuralSums;
    float gh[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const float gz = gc[c] * a.color[c] * (1.f - a.color[c]);
      ga[S::B2 + c] = gz;
#pragma unroll
      for (int h = 0; h < 6; ++h) {
        ga[S::W2 + c * 6 + h] = gz * a.sn[h];
        gh[h] += gz * r[R::W2 + c * 6 + h];
      }
    }
    const float in0 = s[0] / 3.f, in1 = s[1] / 3.f;
#pragma unroll
    for (int h = 0; h < 6; ++h) {
      const float gz = gh[h] * 30.f * a.c[h];
      ga[S::B1 + h] = gz;
      ga[S::W01 + 2 * h + 0] = gz * in0;
      ga[S::W01 + 2 * h + 1] = gz * in1;
      gs[0] += gz * r[R::U + h];
      gs[1] += gz * r[R::V + h];
    }
  } else {
    // colour_c = h1 c1_c + h2 c2_c with h1/h2 = W/2 +/- S, S = sum_f HW_f cos_f.
    // Factors that are constant over the record stay out of the per-pixel
    // terms: ga receives the summands of the pixel sums listed at
    // classic_appearance_gradient, which applies them once per record.
    using R = ClassicRow;
    float g_diff = 0.f;
#pragma unroll
    for (int c = 0; c < 3; ++c) g_diff += gc[c] * r[R::DIFF + c];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      ga[c] = gc[c];
      ga[3 + c] = gc[c] * a.S;
    }
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      ga[6 + f] = a.c[f] * g_diff;
      // d/d(phase_f) = -HW_f sin_f g_diff, phase in radians; the magnitude
      // and local-coordinate derivatives carry 2 pi (revolutions) times dt/d.
      const float gq = a.sn[f] * g_diff;
      // Wave 0 runs along x (direction (1, 0)): its dot product is s[0].
      ga[10 + f] = gq * (f == 0 ? s[0] : kDirX[f] * s[0] + kDirY[f] * s[1]);
      ga[14 + f] = gq;
      gs[0] += gq * r[R::AP + f];
      gs[1] += gq * r[R::BP + f];
    }
  }
}

// The neural output gradients of one record from its reduced sums (NG
// geometry values, the appearance sums laid out as NeuralSums, opacity
// last), written to out[0..kGeometry + kNeural]: geometry columns 0..13; the
// direction, 14..16, sum_h W1[h][2 + k] B1_h; appearance columns 0..56,
// where input weight [h][2 + k] is d_k B1_h and the rest are sums; then the
// opacity. B1_h, the input-bias sum, is the sum over pixels of gz_h, so
// these per-record products equal the per-pixel sums of gz_h W1[h][2 + k]
// and gz_h d_k. out may be the record's own row: its direction and
// direction columns are read before anything is written.
__device__ __forceinline__ void neural_outputs(const float* sums, float* out) {
  using R = NeuralRow;
  using S = NeuralSums;
  constexpr int NG = Layout<true>::NG;
  float wdir[18], dir[3], b1[6];
#pragma unroll
  for (int i = 0; i < 18; ++i) wdir[i] = out[R::WDIR + i];
#pragma unroll
  for (int k = 0; k < 3; ++k) dir[k] = out[R::DIR + k];
#pragma unroll
  for (int h = 0; h < 6; ++h) b1[h] = sums[NG + S::B1 + h];
#pragma unroll
  for (int p = 0; p < NG; ++p) out[p] = sums[p];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    float v = 0.f;
#pragma unroll
    for (int h = 0; h < 6; ++h) v += wdir[h * 3 + k] * b1[h];
    out[NG + k] = v;
  }
  float* app = out + kGeometry;
#pragma unroll
  for (int h = 0; h < 6; ++h) {
    app[5 * h + 0] = sums[NG + S::W01 + 2 * h + 0];
    app[5 * h + 1] = sums[NG + S::W01 + 2 * h + 1];
#pragma unroll
    for (int k = 0; k < 3; ++k) app[5 * h + 2 + k] = dir[k] * b1[h];
  }
#pragma unroll
  for (int h = 0; h < 6; ++h) app[30 + h] = b1[h];
#pragma unroll
  for (int i = 0; i < 21; ++i) app[36 + i] = sums[NG + S::W2 + i];  // output weights, then biases
  app[kNeural] = sums[Layout<true>::NP - 1];
}

// Gradient of classic appearance column k of one record from the pixel
// sums that the classic adjoint accumulates (shade_backward):
//   k 0-2   sum gc_c                -> colour_c   = W/2 sum gc_c + sum gc_c S
//   k 3-5   sum gc_c S              -> colour2_c  = W/2 sum gc_c - sum gc_c S
//   k 6-9   sum cos_f g_diff        -> weight_f   = (sum_c SUM_c sum gc_c + sum) / 2
//   k 10-13 sum sin_f g_diff dot_f  -> magnitude_f = -2 pi HW_f sum
//   k 14-17 sum sin_f g_diff        -> phase_f    = -HW_f sum
// (W/2 = sum_f HW_f, SUM_c = c1_c + c2_c, dot_f = the wave direction . s).
__device__ __forceinline__ float classic_appearance_gradient(const float* sums, const float* r,
                                                             int k) {
  using R = ClassicRow;
  if (k < 6) {
    const int c = k < 3 ? k : k - 3;
    return k < 3 ? r[R::HALF_W] * sums[c] + sums[3 + c] : r[R::HALF_W] * sums[c] - sums[3 + c];
  }
  if (k < 10) {
    const float g_sum = r[R::SUM] * sums[0] + r[R::SUM + 1] * sums[1] + r[R::SUM + 2] * sums[2];
    return 0.5f * (g_sum + sums[k]);
  }
  if (k < 14) return -kTwoPi * r[R::HW + k - 10] * sums[k];
  return -r[R::HW + k - 14] * sums[k];
}

// Replay: walk the tile's replay list written by the forward (replay +
// range start, replay_counts[tile] entries) instead of its point list up to
// tile_last[tile], compositing each record only in the quadrants that took
// it; tile_last is then unused.
// Workgroups per CU: the classic replay walk runs six (25.1 KB of LDS each;
// the compiler holds it to 80 VGPRs and spills only outside the record loop,
// which stays free of scratch), the others four, or two for the neural
// full-list walk.
template <bool Neural, bool Replay>
constexpr int backward_occupancy() {
  return Neural ? (Replay ? 4 : 2) : (Replay ? 6 : 4);
}

template <bool Neural, bool Replay>
__global__ __launch_bounds__(kTilePixels, (backward_occupancy<Neural, Replay>())) void renderBackward(
    int width, int height, int tw, int th, const float* __restrict__ geometry,
    const float* __restrict__ appearance, const float* __restrict__ opacities,
    const int64_t* __restrict__ primitive_ids, const float* __restrict__ backgrounds,
    const int* __restrict__ point_list, const int2* __restrict__ ranges,
    const int* __restrict__ order, const int* __restrict__ tile_last,
    const int2* __restrict__ replay, const int* __restrict__ replay_counts,
    const float* __restrict__ state, const int* __restrict__ contributors,
    MapGroups<const float> grad_maps, float near_plane, float far_plane,
    float* __restrict__ grad_geometry, const AppearanceGradient grad_appearance,
    float* __restrict__ grad_opacities, float* __restrict__ grad_backgrounds,
    const int2* __restrict__ segments, Segments seg) {
  using L = Layout<Neural>;
  constexpr int NP = L::NP;
  constexpr int NG = L::NG;
  constexpr int OP = Neural ? NeuralRow::OP : ClassicRow::OP;
  __shared__ __align__(16) float rows[kBatch * L::STRIDE];
  // The raw staging rows are dead once a batch's rows are derived, and the
  // gradient accumulator is needed only after that: they share LDS, which
  // fits four neural replay workgroups in a CU (39.9 KB each).
  constexpr int kRawFloats = kBatch * L::RAW_STRIDE, kAccFloats = kBatch * NP;
  __shared__ __align__(16) float raw_acc[kRawFloats > kAccFloats ? kRawFloats : kAccFloats];
  float* raw = raw_acc;
  float* acc = raw_acc;
  __shared__ float reach_rows[kBatch * kReachPitch];
  __shared__ int ids[kBatch];
  __shared__ int64_t prims[kBatch];
  __shared__ int entries[kBatch];  // replay entries (position | quadrant bits) of the batch
  __shared__ float bg_acc[3];
  // Classic flush: per record, the addresses of its geometry, appearance and
  // opacity gradient rows, each less its first output column.
  __shared__ uint64_t row_bases[Neural ? 1 : 3 * kBatch];
  const int lane = lane_id();
  // (tile, segment) of this workgroup; past the segment count: nothing.
  const int2 piece = segments ? segments[blockIdx.x] : make_int2(order[blockIdx.x], 0);
  if (piece.x < 0) return;
  const int tile = piece.x;
#ifdef GS_DIAGNOSTICS
  const long long diag_begin = wall_clock64();
  __shared__ unsigned int diag_lanes[65];
  __shared__ unsigned int diag_packing[5];
  for (int i = threadIdx.x; i < 65; i += kTilePixels) diag_lanes[i] = 0u;
  if (threadIdx.x < 5) diag_packing[threadIdx.x] = 0u;
  PackingCounts packing;
#endif
  const TilePixel tp = tile_pixel(tile, width, height, tw, th);
  const float x = float(tp.px), y = float(tp.py);
  const int wave = threadIdx.x >> 6;
  const float tile_x = float(tp.px - (wave & 1) * 8 - (lane & 7));
  const float tile_y = float(tp.py - (wave >> 1) * 8 - (lane >> 3));
  const int last = tp.inside ? contributors[tp.pixel] : 0;

  if (threadIdx.x < 3) bg_acc[threadIdx.x] = 0.f;

  float go[kMaps];
#pragma unroll
  for (int c = 0; c < kMaps; ++c) {
    const float* g = grad_maps.data[map_group(c)];  // null: no gradient for the group
    go[c] = (tp.inside && g) ? g[grad_maps.offset(c, tp.pixel)] : 0.f;
  }
  const float final_t = tp.inside ? state[tp.pixel * 3 + 0] : 0.f;
  const float m1 = tp.inside ? state[tp.pixel * 3 + 1] : 0.f;
  const float m2 = tp.inside ? state[tp.pixel * 3 + 2] : 0.f;
  const float total_a = 1.f - final_t;
  float T = final_t;
  float background_dot = 0.f;
#pragma unroll
  for (int c = 0; c < 3; ++c) background_dot += go[c] * backgrounds[tp.image * 3 + c];
  // dL/dalpha_i picks up final_t (go_alpha - background . go_rgb) / (1 - alpha_i).
  const float final_term = final_t * (go[3] - background_dot);
  // Records walked backwards: list positions up to the tile's largest
  // contributor count, or the replay list's entries [block_first,
  // block_last) - all of them, or one segment's of a split tile, which
  // starts from checkpoint c_{k+1}: its transmittance, and the suffix
  // sum_{later records} w dL/dw from c_K - c_{k+1} (the map gradients weigh
  // the prefix-sum differences; distortion through the final m1, m2).
  const int2 range = ranges[tile];
  int block_first = 0;
  int block_last = Replay ? replay_counts[tile] : tile_last[tile];
  float suffix = 0.f;
  if (Replay && seg.length > 0 && seg.index[tile] >= 0) {
    const int base = seg.index[tile];
    const int pieces = segment_count(range.y - range.x, seg.length);
    const int* n = seg.index + seg.tiles + base;
    block_first = piece.y ? n[piece.y - 1] : 0;
    block_last = n[piece.y];
    if (piece.y < pieces - 1 && tp.inside) {
      constexpr int kSlot = kCheckpointFloats * kTilePixels;
      const float* c = seg.state + int64_t(base + piece.y) * kSlot + threadIdx.x;
      const float* f = seg.state + int64_t(base + pieces - 1) * kSlot + threadIdx.x;
      float d[10];  // T, rgb, depth, normals, m1, m2
#pragma unroll
      for (int q = 0; q < 10; ++q) d[q] = f[q * kTilePixels] - c[q * kTilePixels];
      T = c[0];
      suffix = go[0] * d[1] + go[1] * d[2] + go[2] * d[3] + go[4] * d[4] + go[5] * d[5] +
               go[6] * d[6] + go[7] * d[7] +
               go[8] * (total_a * d[9] - m2 * d[0] - 2.f * m1 * d[8]);
    }
  }
  // Whether every map gradient and saved state value of the wave's pixels is
  // finite (selects the adjoint without per-lane masking).
  bool finite = isfinite(final_term) && isfinite(m1) && isfinite(m2) && isfinite(T) &&
                isfinite(suffix);
#pragma unroll
  for (int c = 0; c < kMaps; ++c) finite = finite && isfinite(go[c]);
  const bool finite_pixels = __all(finite);
  __syncthreads();
  // Background gradient: sum over the tile of final T * dL/drgb (once per
  // tile: by its first segment).
  if (piece.y == 0) {
    const float gb[3] = {final_t * go[0], final_t * go[1], final_t * go[2]};
    const float total = wave_reduce_quads<3>(gb, lane);
    const int param = rs_quad_param<3>(lane);
    if (param < 3 && total != 0.f) atomicAdd(&bg_acc[param], total);
  }
  // Records past every lane's last contributor are inactive in this wave.
  const int wave_last = __builtin_amdgcn_readfirstlane(wave_max(last));
  const float mscale = far_plane / (far_plane - near_plane);
  const float mnear = mscale * near_plane;
  // Per-pixel factors of the depth and distortion terms of the adjoint, with
  // g4, g8 the depth and distortion map gradients and A = 1 - final T:
  //   g4 depth + g8 (m^2 A + m2 - 2 m m1) = g4 depth + m (a8 m - c8) + d8,
  //   dL/dz = w g4 + 2 w g8 mnear (m A - m1) / depth^2
  //         = w (g4 + (e8 m - f8) / depth^2),
  // a8 = g8 A, c8 = 2 g8 m1, d8 = g8 m2, e8 = 2 a8 mnear, f8 = c8 mnear.
  // They are constant over the tile's records (the masked adjoint derives
  // them from its masked gradients instead).
  struct DepthTerms {
    float a8, c8, d8, e8, f8;
  };
  auto depth_terms = [&](float g8) {
    DepthTerms t;
    t.a8 = g8 * total_a;
    t.c8 = 2.f * g8 * m1;
    t.d8 = g8 * m2;
    t.e8 = 2.f * t.a8 * mnear;
    t.f8 = t.c8 * mnear;
    return t;
  };
  const DepthTerms pixel_terms = depth_terms(go[8]);

  // Record threadIdx.x of a batch starting at `start` is list position (or
  // replay entry) range.x + start - 1 - threadIdx.x; the next batch's entry
  // and id are read ahead as in the forward.
  int next_id = 0, next_entry = 0;
  int64_t next_prim = 0;
  if (int(threadIdx.x) < min(kBatch, block_last - block_first)) {
    if constexpr (Replay) {
      const int2 e = replay[range.x + block_last - 1 - threadIdx.x];
      next_id = e.x;
      next_entry = e.y;
    } else {
      next_id = point_list[range.x + block_last - 1 - threadIdx.x];
    }
    next_prim = primitive_ids[next_id];
  }
  for (int start = block_last; start > block_first; start -= kBatch) {
    const int count = min(kBatch, start - block_first);
    const int id = next_id, entry = next_entry;
    const int64_t prim = next_prim;
    const bool ahead = int(threadIdx.x) < min(kBatch, start - kBatch - block_first);
    if (ahead) {
      if constexpr (Replay) {
        const int2 e = replay[range.x + start - kBatch - 1 - threadIdx.x];
        next_id = e.x;
        next_entry = e.y;
      } else {
        next_id = point_list[range.x + start - kBatch - 1 - threadIdx.x];
      }
    }
    const uint64_t reach = load_batch<Neural, Replay ? kReplayMask : kReachTest>(
        rows, raw, reach_rows, ids, prims, tile_x, tile_y, count, id, prim, geometry, appearance,
        opacities, entry, entries);
    if (ahead) next_prim = primitive_ids[next_id];
    // The raw rows are dead: clear the accumulator that shares their LDS
    // (16-byte stores; the array is 16-byte aligned).
    {
      const int n = count * NP;
      float4* acc4 = reinterpret_cast<float4*>(acc);
      for (int i = threadIdx.x; i < n / 4; i += kTilePixels)
        acc4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (int(threadIdx.x) < (n & 3)) acc[(n & ~3) + threadIdx.x] = 0.f;
    }
    __syncthreads();
    uint64_t todo = wave_uniform(reach);
    if constexpr (!Replay) {
      // Row j holds list position start - j (counted from 1).
      const int beyond = start - wave_last;  // rows j < beyond lie past wave_last
      if (beyond >= 64) todo = 0;
      else if (beyond > 0) todo &= ~((uint64_t(1) << beyond) - 1);
    }
    // Whether the wave's gradients and state are finite is constant over the
    // tile, so the record loop is compiled once per adjoint variant and no
    // per-record branch splits it.
    auto walk = [&](auto masked) {
    while (todo) {
      const int j = __builtin_ctzll(todo);
      todo &= todo - 1;
      const float* r = rows + j * L::STRIDE;
      // List position of row j, counted from 1.
      int position = start - j;
      if constexpr (Replay)
        position = __float_as_int(r[Neural ? NeuralRow::POS : ClassicRow::POS]) + 1;
      // A replayed record was taken in the forward by a pixel of this wave's
      // quadrant, so some lane accepts it again and the wave-wide tests are
      // skipped (were none to accept, the stand-ins would make the adjoint
      // add zeros). The full list walk keeps them.
      // position >= 1 and last = 0 outside the image, so the comparison
      // alone keeps those lanes out (no branch around the position's load).
      Sample v;
      const bool active = sample_surface<Neural, true, !Replay>(r, x, y, near_plane,
                                                               position <= last, v);
      if constexpr (!Replay) {
        if (!__any(active)) continue;
      }
#ifdef GS_DIAGNOSTICS
      {
        const uint64_t taking = __ballot(active);
        if (lane == 0 && taking) atomicAdd(&diag_lanes[__popcll(taking)], 1u);
        if (taking) packing.add(taking);
      }
#endif
      // Every lane runs the adjoint. A lane that does not take the sample
      // contributes exact zeros: the sample's values are finite stand-ins
      // (alpha, e, s and 1/p_z zero, depth one), so its weight w and every
      // term carrying e or 1/p_z vanish, and with finite map gradients and
      // pixel state every term below is a product with a zero. A wave with
      // a non-finite one (0 * inf) takes the Masked copy, which also zeroes
      // the lane's map gradients and dL/dalpha. Taking lanes compute exactly
      // what a branch would; the stand-ins replace zero-filling all NP
      // values ahead of a divergent branch.
      auto adjoint = [&](auto masked) {
        constexpr bool kMasked = decltype(masked)::value;
        float gom[kMaps];
#pragma unroll
        for (int c = 0; c < kMaps; ++c) gom[c] = kMasked ? (active ? go[c] : 0.f) : go[c];
        const float alpha = v.alpha;
        const float depth = v.depth;
        const float e = v.e;
        const float inv_pz = v.inv_pz;
        const float s_[2] = {v.s[0], v.s[1]};
        const bool surface = v.surface;
        float grad[NP];  // geometry NG | appearance A | opacity
        float* gg = grad;
        float* ga = grad + NG;
        const float inv_keep = rcp(1.f - alpha);
        T *= inv_keep;  // alpha = 0, inv_keep = 1 where the lane does not take the sample
        const float w = T * alpha;
        Shade a;
        shade<Neural, true>(r, s_, a);
        const DepthTerms dt = kMasked ? depth_terms(gom[8]) : pixel_terms;
        const float inv_depth = rcp(depth);
        const float m = mscale - mnear * inv_depth;
        float gw = gom[4] * depth + (m * (dt.a8 * m - dt.c8) + dt.d8);
        float gc[3];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          // One accumulation per term: a chain of fused multiply-adds.
          gw += gom[c] * a.color[c];
          gw += gom[5 + c] * r[11 + c];
          gc[c] = w * gom[c];
          gg[11 + c] = w * gom[5 + c];
        }
        const float galpha_lane = T * gw + (final_term - suffix) * inv_keep;
        const float galpha = kMasked ? (active ? galpha_lane : 0.f) : galpha_lane;
        suffix += w * gw;
        float gs[2] = {0.f, 0.f};
        shade_backward<Neural>(r, s_, a, gc, ga, gs);
        const float gz = w * (gom[4] + (dt.e8 * m - dt.f8) * (inv_depth * inv_depth));
        // The depth tilts with s only where a classic sample lies on the surface.
        const float gz_tilt = (Neural || surface) ? gz : 0.f;
        gs[0] += gz_tilt * r[6];
        gs[1] += gz_tilt * r[7];
        gg[6] = gz_tilt * s_[0];
        gg[7] = gz_tilt * s_[1];
        gg[8] = gz;
        // alpha = min(0.99, o e) is below the clamp exactly when o e < 0.99
        // (stand-in lanes: alpha = e = 0). Below it, dL/do = galpha e and
        // dL/drho = -o galpha e / 2; g2 is twice the latter.
        const bool below = alpha < 0.99f;
        const float ge = below ? galpha * e : 0.f;
        grad[NP - 1] = ge;
        const float g2 = -r[OP] * ge;
        // rho is rho3 = |s|^2 on the surface (d/ds = 2 s) and otherwise
        // rho2 = 2 |xy - pixel|^2 (d/dxy = 4 (xy - pixel)).
        const float grho3 = surface ? g2 : 0.f;
        const float grho2 = surface ? 0.f : 2.f * g2;
        gs[0] += s_[0] * grho3;
        gs[1] += s_[1] * grho3;
        gg[9] = (r[9] - x) * grho2;
        gg[10] = (r[10] - y) * grho2;
        const float gp[3] = {gs[0] * inv_pz, gs[1] * inv_pz,
                             -(gs[0] * s_[0] + gs[1] * s_[1]) * inv_pz};
        // p = k x l  =>  dk = l x gp, dl = gp x k; k = x T2 - T0 and l = y T2 - T1,
        // so the T rows receive -dk, -dl and x dk + y dl: computed directly as
        // gp x l = -dk and k x gp = -dl.
        const float nk[3] = {gp[1] * v.l[2] - gp[2] * v.l[1], gp[2] * v.l[0] - gp[0] * v.l[2],
                             gp[0] * v.l[1] - gp[1] * v.l[0]};
        const float nl[3] = {v.k[1] * gp[2] - v.k[2] * gp[1], v.k[2] * gp[0] - v.k[0] * gp[2],
                             v.k[0] * gp[1] - v.k[1] * gp[0]};
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          gg[k] = nk[k];
          gg[3 + k] = nl[k];
          gg[6 + k] -= x * nk[k] + y * nl[k];
        }
        // Wave totals, one per lane, added into the batch accumulator.
        float* dst = acc + j * NP;
        if constexpr (NP <= 64) {
          const float total = wave_reduce_quads<NP>(grad, lane);
          const int param = rs_quad_param<NP>(lane);
          if (param < NP && total != 0.f) atomicAdd(dst + param, total);
        } else {
          constexpr int H = NP / 2;
          float lo[H], hi[NP - H];
#pragma unroll
          for (int k = 0; k < H; ++k) lo[k] = grad[k];
#pragma unroll
          for (int k = 0; k < NP - H; ++k) hi[k] = grad[H + k];
          const float t0 = wave_reduce_quads<H>(lo, lane);
          const int p0 = rs_quad_param<H>(lane);
          if (p0 < H && t0 != 0.f) atomicAdd(dst + p0, t0);
          const float t1 = wave_reduce_quads<NP - H>(hi, lane);
          const int p1 = rs_quad_param<NP - H>(lane);
          if (p1 < NP - H && t1 != 0.f) atomicAdd(dst + H + p1, t1);
        }
      };
      adjoint(masked);
    }
    };
    if (finite_pixels)
      walk(std::false_type{});
    else
      walk(std::true_type{});
#ifdef GS_DIAGNOSTICS
    packing.flush(diag_packing);
#endif
    __syncthreads();
    // Flush this batch: one global atomic per nonzero (record, parameter).
    // Consecutive threads take consecutive parameters of a record, so that
    // the atomics of a wave fall on a few cache lines.
    // Output parameters per record: geometry (classic columns 0..13, neural
    // all 17), appearance, opacity; each from the record's reduced sums.
    constexpr int NGO = Neural ? kGeometry : NG;
    constexpr int NO = NGO + L::A + 1;
    if constexpr (!Neural) {
      // Classic: the outputs are the sums themselves (acc[j * NP + p], p <
      // NP = NO) but for the appearance columns, which one thread per record
      // turns into gradients in place first, together with the addresses of
      // the record's three gradient rows, each less the first output column
      // it holds. The flush items then take no branch on their column.
      static_assert(NO == NP, "classic outputs are the reduced values");
      if (int(threadIdx.x) < count) {
        const int j = threadIdx.x;
        float* sums = acc + j * NP + NG;
        const float* r = rows + j * L::STRIDE;
        float g[L::A];
#pragma unroll
        for (int k = 0; k < L::A; ++k) g[k] = classic_appearance_gradient(sums, r, k);
#pragma unroll
        for (int k = 0; k < L::A; ++k) sums[k] = g[k];
        const int64_t prim = prims[j];
        row_bases[3 * j + 0] = reinterpret_cast<uint64_t>(grad_geometry) +
                               uint64_t(int64_t(ids[j]) * kGeometry) * sizeof(float);
        row_bases[3 * j + 1] = reinterpret_cast<uint64_t>(grad_appearance.data[0]) +
                               uint64_t(prim * L::A - NG) * sizeof(float);
        row_bases[3 * j + 2] = reinterpret_cast<uint64_t>(grad_opacities) +
                               uint64_t(prim - (NG + L::A)) * sizeof(float);
      }
      __syncthreads();
      for (int idx = threadIdx.x; idx < count * NP; idx += kTilePixels) {
        const float value = acc[idx];
        if (value != 0.f) {
          const int j = idx / NP;
          const int p = idx - j * NP;
          const int group = int(p >= NG) + int(p >= NG + L::A);
          global_add(row_bases[3 * j + group] + uint64_t(p) * sizeof(float), value);
        }
      }
      // The next batch overwrites ids/prims/rows; every flush must finish first.
      __syncthreads();
      continue;
    }
    // Neural: one thread per record writes its NO output gradients over its
    // own row (once the row's direction and direction-column constants are
    // in registers: nothing else reads the row after the walk), so the flush
    // items read them without the per-column branches of the mapping.
    static_assert(NO <= L::STRIDE, "a neural row holds the record's outputs");
    if (int(threadIdx.x) < count) {
      const int j = threadIdx.x;
      neural_outputs(acc + j * NP, rows + j * L::STRIDE);
    }
    __syncthreads();
    {
      // Destination of output p of a record: geometry columns 0..16 of row
      // ids[j], the appearance columns (one [P, 57] row, or the SIREN's four
      // groups) and the opacity of primitive prims[j]. The group bounds are
      // constants, so the address is a chain of selects, not branches.
      const bool columns = grad_appearance.columns;
      for (int idx = threadIdx.x; idx < count * NO; idx += kTilePixels) {
        const int j = idx / NO;
        const int p = idx - j * NO;
        const float value = rows[j * L::STRIDE + p];
        if (value != 0.f) {
          const int a = p - NGO;  // appearance column; geometry below 0, opacity L::A
          const auto address = [](const float* t) { return reinterpret_cast<uint64_t>(t); };
          uint64_t base = address(grad_appearance.data[0]);
          int width = L::A, first = 0;
          if (columns) {
            base = a < 30   ? address(grad_appearance.data[0])
                   : a < 36 ? address(grad_appearance.data[1])
                   : a < 54 ? address(grad_appearance.data[2])
                            : address(grad_appearance.data[3]);
            width = a < 30 ? 30 : a < 36 ? 6 : a < 54 ? 18 : 3;
            first = a < 30 ? 0 : a < 36 ? 30 : a < 54 ? 36 : 54;
          }
          const bool geometry_column = a < 0, opacity = a >= L::A;
          base = geometry_column ? address(grad_geometry) : (opacity ? address(grad_opacities) : base);
          width = geometry_column ? kGeometry : (opacity ? 1 : width);
          first = geometry_column ? -NGO : (opacity ? L::A : first);
          const int64_t row = geometry_column ? int64_t(ids[j]) : prims[j];
          global_add(base + uint64_t(row * width + (a - first)) * sizeof(float), value);
        }
      }
    }
    // The next batch overwrites ids/prims/rows; every flush must finish first.
    __syncthreads();
  }
  __syncthreads();
  if (threadIdx.x < 3 && bg_acc[threadIdx.x] != 0.f)
    atomicAdd(grad_backgrounds + tp.image * 3 + threadIdx.x, bg_acc[threadIdx.x]);
#ifdef GS_DIAGNOSTICS
  if (gs_diagnostics.lanes && threadIdx.x < 65 && diag_lanes[threadIdx.x] != 0u)
    atomicAdd(gs_diagnostics.lanes + threadIdx.x,
              static_cast<unsigned long long>(diag_lanes[threadIdx.x]));
  if (gs_diagnostics.counters && threadIdx.x < 5 && diag_packing[threadIdx.x] != 0u)
    atomicAdd(gs_diagnostics.counters + 2 + threadIdx.x,
              static_cast<unsigned long long>(diag_packing[threadIdx.x]));
  stamp_tile(gs_diagnostics.backward_span, tile, diag_begin);
#endif
}

struct RenderWorkspace {
  int* order;      // [tiles]
  int* tile_last;  // [tiles]: the backward's start per tile; the forward's probed costs
  int2* segments;  // [tiles + segment slots]: the backward's (tile, segment) order
  size_t bytes;
};

RenderWorkspace render_layout(void* base, int64_t tiles, int64_t segment_slots = 0) {
  RenderWorkspace w;
  char* p = static_cast<char*>(base);
  w.order = reinterpret_cast<int*>(p);
  const size_t half = align_up(size_t(tiles) * sizeof(int), 256);
  w.tile_last = reinterpret_cast<int*>(p + half);
  w.segments = segment_slots > 0 ? reinterpret_cast<int2*>(p + 2 * half) : nullptr;
  w.bytes = 2 * half +
            (segment_slots > 0 ? align_up(size_t(tiles + segment_slots) * sizeof(int2), 256) : 0);
  return w;
}

// Checks the split-tile arguments and describes them (length 0: off).
int make_segments(int32_t length, float* state, int32_t* index, int64_t capacity,
                  int64_t tiles, Segments* seg) {
  *seg = Segments{0, int(tiles), 0, nullptr, nullptr, nullptr};
  if (length == 0) return GS_OK;
  GS_REQUIRE(length > 0 && length % kBatch == 0, GS_ERR_ARGUMENT,
             "segment length must be a positive multiple of %d, got %d", kBatch, length);
  GS_REQUIRE(state && index, GS_ERR_ARGUMENT, "null segment buffers");
  GS_REQUIRE(capacity > 0 && tiles + capacity <= INT_MAX &&
                 capacity <= INT64_MAX / (kCheckpointFloats * kTilePixels * 4),
             GS_ERR_OVERFLOW, "invalid segment capacity %lld for %lld tiles",
             static_cast<long long>(capacity), static_cast<long long>(tiles));
  *seg = Segments{length, int(tiles), int(capacity), state, index,
                  reinterpret_cast<int2*>(index + segment_work_offset(tiles, capacity))};
  return GS_OK;
}

template <typename T>
MapGroups<T> map_groups(T* const* data, const int64_t* strides) {
  MapGroups<T> m;
  for (int g = 0; g < kMapGroups; ++g) {
    m.data[g] = data[g];
    m.pixel_stride[g] = strides[2 * g];
    m.channel_stride[g] = strides[2 * g + 1];
  }
  return m;
}

int check_render(int64_t images, int width, int height, float near_plane, float far_plane) {
  GS_REQUIRE(width > 0 && height > 0 && width < INT_MAX - kTile && height < INT_MAX - kTile,
             GS_ERR_ARGUMENT, "invalid image dimensions");
  GS_REQUIRE(near_plane > 0.f && far_plane > near_plane, GS_ERR_ARGUMENT,
             "invalid clipping planes");
  GS_REQUIRE(images >= 1, GS_ERR_ARGUMENT, "invalid backgrounds");
  GS_REQUIRE(images * tiles_x(width) * tiles_y(height) <= INT_MAX, GS_ERR_OVERFLOW,
             "image tile count exceeds int32");
  return GS_OK;
}

}  // namespace
}  // namespace gs

// Scratch of gs_render_forward_static: the tile dispatch order of up to
// kStaticOrderTiles tiles (4 MiB), one copy per GPU, held until the process
// ends. Host code must not pass `scratch` itself to a kernel (it names the
// host-side shadow, not device memory): the device address comes from
// hipGetSymbolAddress, once per device, in static_order_buffer.
constexpr int64_t kStaticOrderTiles = GS_RENDER_STATIC_MAX_TILES;
static __device__ __align__(256) int scratch[kStaticOrderTiles];

namespace gs {
namespace {

constexpr int kMaxDevices = 64;

// Device address of `scratch` on the device that owns `stream`, looked up
// with that device current on the first call for the device and kept.
int static_order_buffer(hipStream_t stream, int** buffer) {
  static std::mutex mutex;
  static int* addresses[kMaxDevices] = {};
  int current = 0;
  GS_HIP(hipGetDevice(&current));
  int device = current;
  if (stream) GS_HIP(hipStreamGetDevice(stream, &device));
  GS_REQUIRE(device >= 0 && device < kMaxDevices, GS_ERR_ARGUMENT,
             "device %d is beyond the %d devices the static scratch supports", device,
             kMaxDevices);
  std::lock_guard<std::mutex> lock(mutex);
  if (!addresses[device]) {
    if (device != current) GS_HIP(hipSetDevice(device));
    void* address = nullptr;
    const hipError_t found = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (device != current) GS_HIP(hipSetDevice(current));
    GS_HIP(found);
    GS_REQUIRE(address, GS_ERR_HIP, "hipGetSymbolAddress returned no address for the scratch");
    addresses[device] = static_cast<int*>(address);
  }
  *buffer = addresses[device];
  return GS_OK;
}

// The forward compositor's launches given the tile dispatch-order buffer
// (`tiles` ints): gs_render_forward takes it from the caller's workspace,
// gs_render_forward_static from `scratch`.
int render_forward(int32_t neural, const float* geometry, const float* appearance,
                   const float* opacities, const int64_t* primitive_ids,
                   const float* backgrounds, const int32_t* point_list, const int32_t* ranges,
                   int64_t images, int32_t width, int32_t height, float near_plane,
                   float far_plane, const MapGroups<float>& out, float* state,
                   int32_t* contributors, int32_t* replay, int32_t* replay_counts, int* order,
                   int* probe, const Segments& seg, hipStream_t s) {
  ProfileScope prof(GS_PROF_RENDER_FWD, s);
  const int tw = tiles_x(width), th = tiles_y(height);
  const int tiles = int(images * tw * th);
  const int2* r = reinterpret_cast<const int2*>(ranges);
  // Few rounds of workgroups: order by the probed walk lengths instead of
  // the list lengths (tile_probe_kernel).
  const bool probed = probe && !seg.length && tiles <= kProbeMaxTiles;
  if (probed) {
    auto run = [&](auto kernel) {
      kernel<<<unsigned(ceil_div(tiles, 256 / 64)), 256, 0, s>>>(
          tiles, width, height, tw, th, geometry, opacities, primitive_ids, point_list, r,
          near_plane, probe);
    };
    if (neural) run(tile_probe_kernel<true>);
    else run(tile_probe_kernel<false>);
    GS_LAUNCHED("tile_probe_kernel");
  }
  tile_order_kernel<<<1, kOrderBlock, 0, s>>>(probed ? probe : nullptr, r, tiles, order, seg);
  GS_LAUNCHED("tile_order_kernel");
  int2* lists = reinterpret_cast<int2*>(replay);
  const unsigned blocks = unsigned(seg.length ? tiles + seg.capacity : tiles);
  auto launch = [&](auto kernel) {
    kernel<<<blocks, kTilePixels, 0, s>>>(
        width, height, tw, th, geometry, appearance, opacities, primitive_ids, backgrounds,
        point_list, r, order, near_plane, far_plane, out, state, contributors, lists,
        replay_counts, seg);
  };
  if (seg.length) {
    if (neural) {
      if (replay) launch(renderForward<true, true, true>);
      else launch(renderForward<true, false, true>);
    } else {
      if (replay) launch(renderForward<false, true, true>);
      else launch(renderForward<false, false, true>);
    }
  } else {
    if (neural) {
      if (replay) launch(renderForward<true, true, false>);
      else launch(renderForward<true, false, false>);
    } else {
      if (replay) launch(renderForward<false, true, false>);
      else launch(renderForward<false, false, false>);
    }
  }
  GS_LAUNCHED("renderForward");
  if (seg.length) {
    auto merge = [&](auto kernel) {
      kernel<<<unsigned(tiles), kTilePixels, 0, s>>>(
          width, height, tw, th, geometry, appearance, opacities, primitive_ids, backgrounds,
          point_list, r, near_plane, far_plane, out, state, contributors, lists, replay_counts,
          seg);
    };
    if (neural) merge(mergeSegments<true>);
    else merge(mergeSegments<false>);
    GS_LAUNCHED("mergeSegments");
  }
  return GS_OK;
}

// The backward's appearance gradient argument: rows, or (neural only) the
// SIREN's four column groups (a group of no primitives may be null).
int make_appearance_gradient(int32_t neural, float* rows, float* const* columns,
                             AppearanceGradient* out) {
  *out = AppearanceGradient{{rows, nullptr, nullptr, nullptr}, false};
  if (!columns) return GS_OK;
  GS_REQUIRE(neural, GS_ERR_ARGUMENT, "appearance column groups are for the neural renderer");
  for (int g = 0; g < 4; ++g) out->data[g] = columns[g];
  out->columns = true;
  return GS_OK;
}

// Argument checks shared by both forward entry points.
int check_render_forward(int64_t images, int32_t width, int32_t height, float near_plane,
                         float far_plane, const float* backgrounds, const int32_t* ranges,
                         float* const* maps, const int64_t* map_strides, const float* state,
                         const int32_t* contributors, const int32_t* replay,
                         int64_t replay_capacity, const int32_t* replay_counts) {
  int status = check_render(images, width, height, near_plane, far_plane);
  if (status != GS_OK) return status;
  GS_REQUIRE(backgrounds && ranges && maps && map_strides && state && contributors,
             GS_ERR_ARGUMENT, "null pointer passed to gs_render_forward");
  GS_REQUIRE(!replay == !replay_counts, GS_ERR_ARGUMENT,
             "replay and replay_counts must both be given or both be null");
  GS_REQUIRE(!replay || (replay_capacity >= 0 && replay_capacity <= kReplayPositionMask),
             GS_ERR_OVERFLOW, "replay lists need a point list of at most %d entries, got %lld",
             kReplayPositionMask, static_cast<long long>(replay_capacity));
  for (int g = 0; g < kMapGroups; ++g)
    GS_REQUIRE(maps[g], GS_ERR_ARGUMENT, "null map output group %d", g);
  return GS_OK;
}

}  // namespace
}  // namespace gs

extern "C" {

size_t gs_render_workspace_size(int64_t images, int32_t width, int32_t height) {
  if (images < 0 || width <= 0 || height <= 0) return 256;
  return gs::render_layout(nullptr, images * gs::tiles_x(width) * gs::tiles_y(height)).bytes + 256;
}

size_t gs_render_backward_workspace_size(int64_t images, int32_t width, int32_t height,
                                         int64_t segment_capacity) {
  if (images < 0 || width <= 0 || height <= 0 || segment_capacity < 0) return 256;
  const int64_t tiles = images * gs::tiles_x(width) * gs::tiles_y(height);
  return gs::render_layout(nullptr, tiles, segment_capacity).bytes + 256;
}

int gs_render_forward(int32_t neural, const float* geometry, const float* appearance,
                      const float* opacities, const int64_t* primitive_ids,
                      const float* backgrounds, const int32_t* point_list,
                      const int32_t* ranges, int64_t images, int32_t width, int32_t height,
                      float near_plane, float far_plane, float* const* maps,
                      const int64_t* map_strides, float* state, int32_t* contributors,
                      int32_t* replay, int64_t replay_capacity, int32_t* replay_counts,
                      int32_t segment_length, float* segment_state, int32_t* segment_index,
                      int64_t segment_capacity, void* workspace, size_t workspace_bytes,
                      void* stream) {
  using namespace gs;
  clear_error();
  int status =
      check_render_forward(images, width, height, near_plane, far_plane, backgrounds, ranges,
                           maps, map_strides, state, contributors, replay, replay_capacity,
                           replay_counts);
  if (status != GS_OK) return status;
  const int64_t tiles = images * tiles_x(width) * tiles_y(height);
  Segments seg;
  status = make_segments(segment_length, segment_state, segment_index, segment_capacity,
                         tiles, &seg);
  if (status != GS_OK) return status;
  const size_t need = gs_render_workspace_size(images, width, height);
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE,
             "render forward needs %zu workspace bytes, got %zu", need, workspace_bytes);
  RenderWorkspace w = render_layout(workspace, tiles);
  return render_forward(neural, geometry, appearance, opacities, primitive_ids, backgrounds,
                        point_list, ranges, images, width, height, near_plane, far_plane,
                        map_groups(maps, map_strides), state, contributors, replay,
                        replay_counts, w.order, w.tile_last, seg,
                        static_cast<hipStream_t>(stream));
}

int gs_render_forward_static(int32_t neural, const float* geometry, const float* appearance,
                             const float* opacities, const int64_t* primitive_ids,
                             const float* backgrounds, const int32_t* point_list,
                             const int32_t* ranges, int64_t images, int32_t width,
                             int32_t height, float near_plane, float far_plane,
                             float* const* maps, const int64_t* map_strides, float* state,
                             int32_t* contributors, int32_t* replay, int64_t replay_capacity,
                             int32_t* replay_counts, void* stream) {
  using namespace gs;
  clear_error();
  const int status =
      check_render_forward(images, width, height, near_plane, far_plane, backgrounds, ranges,
                           maps, map_strides, state, contributors, replay, replay_capacity,
                           replay_counts);
  if (status != GS_OK) return status;
  const int64_t tiles = images * tiles_x(width) * tiles_y(height);
  GS_REQUIRE(tiles <= kStaticOrderTiles, GS_ERR_WORKSPACE,
             "gs_render_forward_static handles at most %lld image tiles (its static scratch), "
             "got %lld",
             static_cast<long long>(kStaticOrderTiles), static_cast<long long>(tiles));
  hipStream_t s = static_cast<hipStream_t>(stream);
  int* order = nullptr;
  const int found = static_order_buffer(s, &order);
  if (found != GS_OK) return found;
  return render_forward(neural, geometry, appearance, opacities, primitive_ids, backgrounds,
                        point_list, ranges, images, width, height, near_plane, far_plane,
                        map_groups(maps, map_strides), state, contributors, replay,
                        replay_counts, order, nullptr,
                        Segments{0, int(tiles), 0, nullptr, nullptr, nullptr}, s);
}

int gs_render_backward(int32_t neural, const float* geometry, const float* appearance,
                       const float* opacities, const int64_t* primitive_ids,
                       const float* backgrounds, const int32_t* point_list,
                       const int32_t* ranges, const float* state,
                       const int32_t* contributors, const int32_t* replay,
                       const int32_t* replay_counts, int32_t segment_length,
                       const float* segment_state, const int32_t* segment_index,
                       int64_t segment_capacity, const float* const* grad_maps,
                       const int64_t* grad_map_strides, int64_t images,
                       int32_t width, int32_t height, float near_plane, float far_plane,
                       float* grad_geometry, float* grad_appearance,
                       float* const* grad_appearance_columns, float* grad_opacities,
                       float* grad_backgrounds, void* workspace, size_t workspace_bytes,
                       void* stream) {
  using namespace gs;
  clear_error();
  int status = check_render(images, width, height, near_plane, far_plane);
  if (status != GS_OK) return status;
  AppearanceGradient grad_rows;
  status = make_appearance_gradient(neural, grad_appearance, grad_appearance_columns,
                                    &grad_rows);
  if (status != GS_OK) return status;
  GS_REQUIRE(backgrounds && ranges && state && contributors && grad_maps && grad_map_strides &&
                 grad_backgrounds,
             GS_ERR_ARGUMENT, "null pointer passed to gs_render_backward");
  GS_REQUIRE(!replay == !replay_counts, GS_ERR_ARGUMENT,
             "replay and replay_counts must both be given or both be null");
  const MapGroups<const float> grads = map_groups(grad_maps, grad_map_strides);
  const int tw = tiles_x(width), th = tiles_y(height);
  const int tiles = int(images * tw * th);
  Segments seg;
  status = make_segments(segment_length, const_cast<float*>(segment_state),
                         const_cast<int32_t*>(segment_index), segment_capacity, tiles, &seg);
  if (status != GS_OK) return status;
  GS_REQUIRE(!seg.length || replay, GS_ERR_ARGUMENT,
             "the backward of split tiles needs the replay lists");
  const size_t need =
      gs_render_backward_workspace_size(images, width, height, seg.length ? seg.capacity : 0);
  GS_REQUIRE(workspace && workspace_bytes >= need, GS_ERR_WORKSPACE,
             "render backward needs %zu workspace bytes, got %zu", need, workspace_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfileScope prof(GS_PROF_RENDER_BWD, s);
  const int2* r = reinterpret_cast<const int2*>(ranges);
  RenderWorkspace w = render_layout(workspace, tiles, seg.length ? seg.capacity : 0);
  // Tiles (or the segments of split tiles) are ordered by the records they
  // replay: the replay list's length, or the largest contributor count.
  unsigned blocks = unsigned(tiles);
  if (seg.length) {
    segment_order_kernel<<<1, kOrderBlock, 0, s>>>(r, replay_counts, tiles, seg, w.segments);
    GS_LAUNCHED("segment_order_kernel");
    blocks = unsigned(tiles + seg.capacity);
  } else {
    if (!replay) {
      tile_last_kernel<<<unsigned(tiles), kTilePixels, 0, s>>>(width, height, tw, th,
                                                               contributors, w.tile_last);
      GS_LAUNCHED("tile_last_kernel");
    }
    tile_order_kernel<<<1, kOrderBlock, 0, s>>>(replay ? replay_counts : w.tile_last, r, tiles,
                                                w.order, seg);
    GS_LAUNCHED("tile_order_kernel");
  }
  const int2* lists = reinterpret_cast<const int2*>(replay);
  auto launch = [&](auto kernel) {
    kernel<<<blocks, kTilePixels, 0, s>>>(
        width, height, tw, th, geometry, appearance, opacities, primitive_ids, backgrounds,
        point_list, r, w.order, w.tile_last, lists, replay_counts, state, contributors, grads,
        near_plane, far_plane, grad_geometry, grad_rows, grad_opacities,
        grad_backgrounds, w.segments, seg);
  };
  if (neural) {
    if (replay) launch(renderBackward<true, true>);
    else launch(renderBackward<true, false>);
  } else {
    if (replay) launch(renderBackward<false, true>);
    else launch(renderBackward<false, false>);
  }
  GS_LAUNCHED("renderBackward");
  return GS_OK;
}

int gs_diagnostics_query(int32_t* available, int32_t* wall_clock_khz) {
  GS_REQUIRE(available && wall_clock_khz, GS_ERR_ARGUMENT, "null diagnostics query output");
#ifdef GS_DIAGNOSTICS
  *available = 1;
#else
  *available = 0;
#endif
  int device = 0, khz = 0;
  GS_HIP(hipGetDevice(&device));
  GS_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device));
  *wall_clock_khz = khz;
  return GS_OK;
}

int gs_diagnostics_set(unsigned long long* lanes, long long* forward_span,
                       long long* backward_span, int64_t tiles, unsigned long long* counters) {
  GS_REQUIRE(tiles >= 0, GS_ERR_ARGUMENT, "diagnostics tile count must be non-negative");
#ifdef GS_DIAGNOSTICS
  const gs::DiagnosticTargets targets{lanes, forward_span, backward_span, tiles, counters};
  GS_HIP(hipMemcpyToSymbol(HIP_SYMBOL(gs::gs_diagnostics), &targets, sizeof targets));
  return GS_OK;
#else
  (void)lanes;
  (void)forward_span;
  (void)backward_span;
  (void)counters;
  GS_REQUIRE(false, GS_ERR_ARGUMENT,
             "this library was built without diagnostics (libgabor_hip_diag.so has them)");
  return GS_ERR_ARGUMENT;
#endif
}

}  // extern "C"
