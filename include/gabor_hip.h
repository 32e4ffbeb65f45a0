/*
 * gabor_hip.h - C ABI of the MI355X (gfx950) Gabor-surface tile rasterizer.
 *
 * Every entry point takes plain device pointers, element counts and a HIP
 * stream (passed as void*, a hipStream_t), launches its kernels on that
 * stream and returns a status code. Nothing here allocates device memory:
 * buffers whose size depends on data (tile intersections, sort scratch) are
 * sized by the *_workspace_size queries and owned by the caller. No function
 * throws across the ABI; on failure gs_last_error() names the problem.
 *
 * Tensor layouts (all row-major, contiguous, float32 unless stated):
 *   means [S,N,3]  quaternions [S,N,4] (wxyz)  scales [S,N,2]
 *   view_matrices [S,C,4,4] (world->camera)  intrinsics [S,C,3,3]
 *   geometry [Q,17] = T(3x3 row-major) | xy(2) | normal(3) | direction(3)
 *   appearance [P,18] classic: color(3) color2(3) weights(4) magnitudes(4) phases(4)
 *   appearance [P,57] neural: W1(6x5) b1(6) W2(3x6) b2(3)
 *   maps [I,H,W,9] = rgb(3) alpha depth normal(3) distortion
 *   state [I,H,W,3] = final transmittance, m1, m2;  contributors [I,H,W] int32
 *   keys uint64: (image*tw*th + tile_y*tw + tile_x) << 32 | float bits of depth
 *   ranges [I*tw*th, 2] int32 = [first, last) into the sorted list
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   gabor_splatting._C pybind11 module, src/gabor_splatting/csrc/bindings.cpp:5-10,
 *   declared in src/gabor_splatting/csrc/rasterize.h:6-21, and the PyTorch
 *   projection in src/gabor_splatting/rendering.py:156-218.
 */
#ifndef GABOR_HIP_H
#define GABOR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes returned by every entry point. */
#define GS_OK 0
#define GS_ERR_ARGUMENT 1 /* invalid size, pointer or option */
#define GS_ERR_OVERFLOW 2 /* an int32 index space would overflow */
#define GS_ERR_HIP 3      /* a HIP runtime call or launch failed */
#define GS_ERR_WORKSPACE 4 /* caller workspace smaller than required */

/* Message of the last failure on the calling thread ("" if none). */
const char* gs_last_error(void);

/* ABI version, bumped on any signature change. */
int gs_abi_version(void);

/* ------------------------------------------------------------------ */
/* Kernel 1: projection (replaces rendering.py:156-218 project_surfaces,
 * which the reference runs as PyTorch ops) and its adjoint (the reference
 * relies on PyTorch autograd through those ops).                      */

/* Project every (scene, camera, surfel) pair: T = K [Rc tu*su, Rc tv*sv,
 * Rc mu + t], conic centre xy, facing camera-space normal, unit world
 * direction camera->centre and the integer screen radius (0 = culled).
 * Outputs are [S,C,N,*]: transform 9, xy 2, normals 3, directions 3,
 * radii int32. */
int gs_project_forward(const float* means, const float* quaternions, const float* scales,
                       const float* view_matrices, const float* intrinsics, int64_t scenes,
                       int64_t cameras, int64_t n, int32_t width, int32_t height,
                       float near_plane, float far_plane, float* transform, float* xy,
                       float* normals, float* directions, int32_t* radii, void* stream);

/* Scratch bytes needed by gs_project_backward (per-block camera partials). */
size_t gs_project_backward_workspace_size(int64_t scenes, int64_t cameras, int64_t n);

/* Adjoint of gs_project_forward. Any of grad_transform / grad_xy /
 * grad_normals / grad_directions may be NULL (treated as zero). Outputs are
 * overwritten (not accumulated): grad_means [S,N,3], grad_quaternions
 * [S,N,4], grad_scales [S,N,2], grad_view_matrices [S,C,4,4] (last row 0),
 * grad_intrinsics [S,C,3,3]. Per-camera sums use a deterministic two-stage
 * reduction through the workspace. */
int gs_project_backward(const float* means, const float* quaternions, const float* scales,
                        const float* view_matrices, const float* intrinsics, int64_t scenes,
                        int64_t cameras, int64_t n, const float* grad_transform,
                        const float* grad_xy, const float* grad_normals,
                        const float* grad_directions, float* grad_means,
                        float* grad_quaternions, float* grad_scales,
                        float* grad_view_matrices, float* grad_intrinsics, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Fused projection, SH and compositor-record assembly. Replaces the
 * reference's host chain rendering.py:323-374 (project_surfaces, SHColors,
 * per-camera expansion of shared appearance/opacity, packing gathers and the
 * geometry torch.cat). For every (scene, camera, surfel) pair it writes
 * dense_radii[pair] (if non-null) and, unless geometry is null (a radii-only
 * pass), the pair's compositor row: row = pair when row_of_pair is null,
 * else row_of_pair[pair] (-1: skipped). Rows: geometry [Q,17],
 * projected_means [Q,2], row_radii [Q], image_ids [Q] (= s*C + c),
 * primitive_ids [Q] (= s*N + n without SH; = row with SH). With
 * sh_degree 0..3 the colours are camera-specific and the row also gets
 * appearance_rows [Q,18] (SH colours, then the surfel's weights, magnitudes
 * and phases) and opacity_rows [Q]; sh_degree -1 writes neither (the caller
 * supplies per-surfel appearance). Rows of pairs with radius 0 (referenced
 * by no tile list) get their radius, projected mean and ids; their geometry
 * and appearance rows are zero in dense mode (row_of_pair null) and their
 * opacity entry is left as it was. When
 * given (all three or none), meta_scene_ids / meta_camera_ids /
 * meta_surfel_ids [Q] int64 receive each row's scene, camera and surfel
 * index: the reference's meta ids (rendering.py:389-392). */
int gs_records_forward(const float* means, const float* quaternions, const float* scales,
                       const float* opacities, const float* view_matrices,
                       const float* intrinsics, const float* sh_first, const float* sh_second,
                       const float* frequency_weights, const float* frequency_magnitudes,
                       const float* phases, int32_t sh_degree, int64_t scenes,
                       int64_t cameras, int64_t n, int32_t width, int32_t height,
                       float near_plane, float far_plane, const int32_t* row_of_pair,
                       int32_t* dense_radii, float* geometry, float* projected_means,
                       int32_t* row_radii, int64_t* primitive_ids, int64_t* image_ids,
                       float* appearance_rows, float* opacity_rows, int64_t* meta_scene_ids,
                       int64_t* meta_camera_ids, int64_t* meta_surfel_ids, void* stream);

/* Scratch bytes needed by gs_records_backward. */
size_t gs_records_backward_workspace_size(int64_t scenes, int64_t cameras, int64_t n,
                                          int32_t sh_degree);

/* Adjoint of gs_records_forward given the compositor's row gradients:
 * grad_geometry [Q,17] (its xy columns are ignored: the projected-means
 * gradient arrives in grad_projected_means, Q rows of 2 floats that start
 * grad_projected_stride floats apart: 2 for a [Q,2] array, 17 for the xy
 * columns of a [Q,17] one), and with SH
 * grad_appearance_rows [Q,18] and grad_opacity_rows [Q]; any may be null.
 * geometry is the forward's row output (SH reads the directions). Surfel and
 * camera gradients are overwritten: means, quaternions, scales,
 * view_matrices [S,C,4,4], intrinsics [S,C,3,3], and with SH the
 * coefficients [S,N,K,3] x2, weights/magnitudes/phases [S,N,4] and
 * opacities [S,N], each summed over cameras without atomics.
 * grad_view_matrices and grad_intrinsics may both be null (cameras that
 * take no gradient): the camera adjoint and its reduction are then skipped.
 * One null and one not is an argument error. */
int gs_records_backward(const float* means, const float* quaternions, const float* scales,
                        const float* view_matrices, const float* intrinsics,
                        const float* sh_first, const float* sh_second, int32_t sh_degree,
                        int64_t scenes, int64_t cameras, int64_t n,
                        const int32_t* row_of_pair, const float* geometry,
                        const float* grad_geometry, const float* grad_projected_means,
                        int64_t grad_projected_stride, const float* grad_appearance_rows,
                        const float* grad_opacity_rows,
                        float* grad_means, float* grad_quaternions, float* grad_scales,
                        float* grad_view_matrices, float* grad_intrinsics,
                        float* grad_sh_first, float* grad_sh_second, float* grad_weights,
                        float* grad_magnitudes, float* grad_phases, float* grad_opacities,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Replaces _C.evaluate_sh_forward (spherical_harmonics.cu:107-126):
 * colors [S,C,N,6] = max(0.5 + sum_k Y_k(dir) coef[k], 0) for both colour
 * sets first/second [S,N,K,3], K = (degree+1)^2, directions [S,C,N,3]. */
int gs_sh_forward(const float* first, const float* second, const float* directions,
                  float* colors, int64_t scenes, int64_t cameras, int64_t n, int32_t degree,
                  void* stream);

/* Replaces _C.evaluate_sh_backward (spherical_harmonics.cu:129-150).
 * grad_first/grad_second [S,N,K,3] are overwritten with the sum over
 * cameras (no atomics); grad_directions [S,C,N,3] is overwritten. */
int gs_sh_backward(const float* first, const float* second, const float* directions,
                   const float* grad_colors, float* grad_first, float* grad_second,
                   float* grad_directions, int64_t scenes, int64_t cameras, int64_t n,
                   int32_t degree, void* stream);

/* ------------------------------------------------------------------ */
/* Input value contracts (replaces check_values, rendering.py:88-153,
 * which the reference evaluates as a chain of PyTorch ops).           */

/* One bit per violated contract, in the order the reference lists them:
 * bit k (k < GS_CHECK_MAX_TENSORS) = tensors[k] holds a NaN or infinity,
 * then the value contracts below. */
#define GS_CHECK_MAX_TENSORS 16
#define GS_CHECK_SCALES_POSITIVE (1u << 16)        /* scales > 0 */
#define GS_CHECK_OPACITIES_RANGE (1u << 17)        /* 0 <= opacities <= 1 */
#define GS_CHECK_QUATERNIONS_UNIT (1u << 18)       /* |q|^2 close to 1 */
#define GS_CHECK_VIEW_LAST_ROW (1u << 19)          /* view row 3 = [0,0,0,1] */
#define GS_CHECK_INTRINSICS_LAST_ROW (1u << 20)    /* K row 2 = [0,0,1] */
#define GS_CHECK_FOCAL_POSITIVE (1u << 21)         /* fx > 0 and fy > 0 */
#define GS_CHECK_ROTATION_ORTHONORMAL (1u << 22)   /* R^T R close to I */
#define GS_CHECK_ROTATION_DETERMINANT (1u << 23)   /* det R close to +1 */
#define GS_CHECK_WEIGHTS_NONNEGATIVE (1u << 24)    /* frequency_weights >= 0 */
#define GS_CHECK_MAGNITUDES_NONNEGATIVE (1u << 25) /* frequency_magnitudes >= 0 */
#define GS_CHECK_WEIGHTS_SUM (1u << 26)            /* frequency weights sum to 1 */

/* Writes the violated contracts to *violations (a device uint32, cleared
 * by a one-thread launch first) in one launch that reads every value once:
 * finiteness of tensors[0..tensor_count) (sizes[k] floats each); per
 * surfel (quaternions [surfels,4], scales [surfels,2], opacities [surfels],
 * and, when not null, frequency_weights / frequency_magnitudes
 * [surfels,4]); per image
 * (view_matrices [images,4,4], intrinsics [images,3,3]). Closeness is
 * torch.isclose's |x - t| <= atol + |rtol t| in float32: rtol 1e-5 / atol
 * 1e-8 for the last rows, 1e-4 / 1e-4 for the other closeness contracts. */
int gs_check_values(const float* const* tensors, const int64_t* sizes, int32_t tensor_count,
                    const float* quaternions, const float* scales, const float* opacities,
                    const float* frequency_weights, const float* frequency_magnitudes,
                    int64_t surfels, const float* view_matrices, const float* intrinsics,
                    int64_t images, uint32_t* violations, void* stream);

/* ------------------------------------------------------------------ */
/* Kernel 2: visible-pair packing and tile binning.                    */

/* Scratch bytes for gs_pack_visible / gs_count_tiles over `count` items. */
size_t gs_scan_workspace_size(int64_t count);

/* Packed mode (rendering.py:362-364, `arange(Q)[radii > 0]`): writes the
 * ascending indices of pairs with radii > 0 to selected[0..V) and V to
 * *num_selected (a device int64). selected must hold `count` entries.
 * row_of_pair (optional, [count] int32) receives each pair's row in the
 * packed order, or -1 for culled pairs. */
int gs_pack_visible(const int32_t* radii, int64_t count, int64_t* selected,
                    int32_t* row_of_pair, int64_t* num_selected, void* workspace,
                    size_t workspace_bytes, void* stream);

/* countTiles + cub::DeviceScan::InclusiveSum (rasterize.cu:33-40, 459-464):
 * offsets[i] = inclusive prefix sum of each pair's tile-rectangle area
 * (0 when radii[i] <= 0). offsets [count] int64. */
int gs_count_tiles(const float* geometry, const int32_t* radii, int64_t count, int32_t width,
                   int32_t height, int64_t* offsets, void* workspace, size_t workspace_bytes,
                   void* stream);

/* emitTiles (rasterize.cu:43-56): for each visible pair, one key/value per
 * covered tile in row-major tile order, starting at offsets[i-1].
 * keys/values hold offsets[count-1] entries. */
int gs_emit_tiles(const float* geometry, const int32_t* radii, const int64_t* image_ids,
                  const int64_t* offsets, int64_t count, int32_t width, int32_t height,
                  uint64_t* keys, int32_t* values, void* stream);

/* ------------------------------------------------------------------ */
/* Kernel 3: LSD radix sort and tile ranges.                           */

/* Scratch bytes for gs_sort_pairs over m pairs. */
size_t gs_sort_workspace_size(int64_t m);

/* Stable ascending sort of (key, value) pairs on key bits [begin_bit,
 * end_bit) (cub::DeviceRadixSort::SortPairs, rasterize.cu:478-487). Inputs
 * are not modified; outputs must not alias inputs. */
int gs_sort_pairs(const uint64_t* keys_in, uint64_t* keys_out, const int32_t* values_in,
                  int32_t* values_out, int64_t m, int32_t begin_bit, int32_t end_bit,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Scratch bytes for gs_sort_pairs32 over m pairs. */
size_t gs_sort32_workspace_size(int64_t m);

/* The same stable sort for 32-bit keys, the sort of both depth-first binning
 * stages (each stands in for part of the 64-bit SortPairs of
 * rasterize.cu:478-487): key bits [begin_bit, end_bit), int32 values, or the
 * keys alone when values_in and values_out are both null. */
int gs_sort_pairs32(const uint32_t* keys_in, uint32_t* keys_out, const int32_t* values_in,
                    int32_t* values_out, int64_t m, int32_t begin_bit, int32_t end_bit,
                    void* workspace, size_t workspace_bytes, void* stream);

/* findRanges (rasterize.cu:59-69): ranges [tiles,2] = [first,last) of each
 * tile's run in sorted_keys; tiles with no entries get (0,0). */
int gs_find_ranges(const uint64_t* sorted_keys, int64_t m, int32_t* ranges, int64_t tiles,
                   void* stream);

/* Depth-first binning: the point list and ranges of emitTiles + the 64-bit
 * cub::DeviceRadixSort::SortPairs + findRanges (rasterize.cu:43-69,
 * 470-501), bit for bit, in two stages. A stable sort of the pairs on their
 * depth bits, emission of each pair's tiles in that order as 32-bit tile
 * ids and a stable sort of those on bits(tiles) bits leaves every tile's
 * entries ordered by (depth bits, pair index), as the 64-bit sort does. */

/* Scratch bytes for gs_bin_order over `count` pairs. */
size_t gs_bin_order_workspace_size(int64_t count);

/* Stage 1, which needs no intersection count and so can run while the host
 * waits for it: each pair's tile rectangle (tileBounds, rasterize.cu:24-30)
 * and area (countTiles, :33-40), the stable depth-bit order of the pairs,
 * order [count] int32 (pair at depth rank j), starts [count] int64 (first
 * entry of rank j: entries of all lower ranks), rects [count, 4] int32
 * (x0, y0, width in tiles, image*tw*th, for stage 2) and *intersections
 * (one device int64) = M, the total that rasterize.cu:466-468 copies to the
 * host. *visible (one device int64, or null) receives V, the number of
 * pairs with tiles: they hold depth ranks 0..V-1. */
int gs_bin_order(const float* geometry, const int32_t* radii, const int64_t* image_ids,
                 int64_t count, int32_t width, int32_t height, int32_t* order, int64_t* starts,
                 int32_t* rects, int64_t* intersections, int64_t* visible, void* workspace,
                 size_t workspace_bytes, void* stream);

/* gs_bin_order in two calls, so that the host can read M and V back while
 * the pairs are sorted. No counterpart in the reference, which sums the
 * counts with its scan after countTiles (rasterize.cu:459-469).
 * gs_bin_order_count: the rectangles, counts and depth keys of stage 1,
 * rects as in gs_bin_order, and *intersections = M, *visible = V (null:
 * not wanted), summed as the counts are made. gs_bin_order_sort: the depth
 * order and starts of stage 1 from what gs_bin_order_count left in the same
 * workspace (same count; the workspace untouched in between). */
int gs_bin_order_count(const float* geometry, const int32_t* radii, const int64_t* image_ids,
                       int64_t count, int32_t width, int32_t height, int32_t* rects,
                       int64_t* intersections, int64_t* visible, void* workspace,
                       size_t workspace_bytes, void* stream);
int gs_bin_order_sort(int64_t count, int32_t* order, int64_t* starts, void* workspace,
                      size_t workspace_bytes, void* stream);

/* Scratch bytes for gs_bin_tiles over m intersections. */
size_t gs_bin_tiles_workspace_size(int64_t m);

/* Binning status bits (the `status` word of gs_bin_tiles and the overflow
 * word of gs_bin_tiles_bounded). */
#define GS_BIN_OVERFLOW 1u  /* more intersections than the point list holds */
#define GS_BIN_BAD_INDEX 2u /* a sort produced a rank or pair index outside
                               [0, count); pair 0 was substituted for it */

/* Stage 2 from stage 1's order, starts and rects: emit in depth order,
 * sort by tile id, find ranges. point_list [m] int32, ranges
 * [images*tw*th, 2] int32 ((0,0) for empty tiles). `visible` is stage 1's
 * V, or -1 if unknown: when bits(tiles) + bits(V) <= 32 the entries are
 * sorted as single 32-bit (tile id, depth rank) keys, otherwise as (tile
 * id, pair index) pairs; the result is the same. Every index taken from a
 * sort output is range-checked before it is dereferenced or written to the
 * point list; `status` (a device uint32, or null) is cleared, then gets
 * GS_BIN_BAD_INDEX if a check failed. */
int gs_bin_tiles(const int32_t* order, const int64_t* starts, const int32_t* rects,
                 int64_t count, int64_t m, int64_t visible, int64_t images, int32_t width,
                 int32_t height, int32_t* point_list, int32_t* ranges, uint32_t* status,
                 void* workspace, size_t workspace_bytes, void* stream);

/* Block path: the same point list and ranges as gs_bin_order_count +
 * gs_bin_order_sort + gs_bin_tiles (emitTiles + the 64-bit SortPairs +
 * findRanges, rasterize.cu:43-69, 470-501), bit for bit, with a much
 * smaller sort. No counterpart in the reference. The tiles are grouped in
 * tile blocks of 4 x 4 tiles of one image (row-major per image, image after
 * image). A pair's rectangle meets ~18 tiles but ~3 blocks on a 1080p scene
 * of 1M surfels, so instead of sorting its M tile entries, stage 2 sorts one
 * (block id, 16-bit mask of the block's covered tiles, pair) entry per
 * (pair, block) on the block-id bits, stably, from depth order; then each
 * block's entry list is cut into up to 16 chunks, one wave per chunk counts
 * the entries of each of the block's 16 tiles, a scan of the tile totals
 * gives the ranges, and the same waves write each pair into the lists of
 * the tiles its mask covers, in block-list order, which is (depth bits,
 * pair index) order.
 *
 * gs_bin_blocks_fit: 1 when the block ids of `images` images fit the block
 * path (at most 65536 tile blocks), else 0.
 * gs_bin_blocks_count: stage 1's first step for the block path (the
 * workspace of gs_bin_order_count): rects [count, 4] int32 = (x0, y0 +
 * image*th, x1, y1 + image*th), each pair's tile rectangle with the images'
 * tile rows stacked, and totals [3] int64 on the device = (M, V, E), E the
 * number of (pair, block) entries. Pairs with tiles must have their depth in
 * (near_plane, far_plane), as projection guarantees: for near_plane > 0 the
 * depth keys are then bits(z) - bits(near) (z clamped to [near, far] first),
 * which order the pairs as the raw bits do in bit_length(bits(far) -
 * bits(near) + 1) bits, 27 for (0.2, 100); otherwise the raw 32 bits.
 * gs_bin_blocks_sort, called next with the same workspace and planes, gives
 * the depth order and, as `starts`, the first block entry of each depth rank
 * (gs_bin_order_sort with the depth sort on those bits).
 * gs_bin_blocks_tiles: stage 2 from those order, starts and rects, with M
 * (point_list [m]), E and V (or -1) from totals; ranges and status as in
 * gs_bin_tiles (GS_BIN_OVERFLOW if an entry's slot falls at or past m,
 * which consistent inputs never do). */
int gs_bin_blocks_fit(int64_t images, int32_t width, int32_t height);
int gs_bin_blocks_count(const float* geometry, const int32_t* radii, const int64_t* image_ids,
                        int64_t count, int32_t width, int32_t height, float near_plane,
                        float far_plane, int32_t* rects, int64_t* totals, void* workspace,
                        size_t workspace_bytes, void* stream);
int gs_bin_blocks_sort(int64_t count, float near_plane, float far_plane, int32_t* order,
                       int64_t* starts, void* workspace, size_t workspace_bytes, void* stream);
/* Scratch bytes for gs_bin_blocks_tiles over `entries` block entries. */
size_t gs_bin_blocks_tiles_workspace_size(int64_t entries, int64_t images, int32_t width,
                                          int32_t height);
int gs_bin_blocks_tiles(const int32_t* order, const int64_t* starts, const int32_t* rects,
                        int64_t count, int64_t m, int64_t entries, int64_t visible,
                        int64_t images, int32_t width, int32_t height, int32_t* point_list,
                        int32_t* ranges, uint32_t* status, void* workspace,
                        size_t workspace_bytes, void* stream);

/* gs_bin_tiles without the host's intersection count, for callers that
 * cannot synchronise (HIP graph capture): the point list and workspace are
 * sized for `capacity` entries (point_list [capacity], workspace
 * gs_bin_tiles_workspace_size(capacity)); the live count is read from
 * *intersections, the device word gs_bin_order wrote. The first
 * min(count, capacity) entries of the depth-first emission are binned and
 * ranges cover exactly those; the point-list entries past them are -1. *overflow (a device uint32) is cleared, then
 * gets GS_BIN_OVERFLOW when the count exceeds the capacity (the deepest
 * records were then dropped from their tiles) and GS_BIN_BAD_INDEX as in
 * gs_bin_tiles. No counterpart in the reference, which reads the count on
 * the host (rasterize.cu:466-469). */
int gs_bin_tiles_bounded(const int32_t* order, const int64_t* starts, const int32_t* rects,
                         int64_t count, int64_t capacity, const int64_t* intersections,
                         int64_t images, int32_t width, int32_t height, int32_t* point_list,
                         int32_t* ranges, uint32_t* overflow, void* workspace,
                         size_t workspace_bytes, void* stream);

/* gs_bin_blocks_tiles without the host's counts, for the same callers: the
 * point list holds `capacity` entries and the block entries are sized for
 * as many (E <= M), workspace gs_bin_blocks_tiles_workspace_size(capacity,
 * images, width, height); M and E are read from totals, the device words
 * gs_bin_blocks_count wrote. Within the capacity (M <= capacity) the point
 * list's first M entries and the ranges equal gs_bin_blocks_tiles' and the
 * entries past M are -1. *overflow (a device uint32) is cleared, then gets
 * GS_BIN_OVERFLOW when M exceeds the capacity and GS_BIN_BAD_INDEX as in
 * gs_bin_tiles. On overflow every range stays inside the list and every
 * entry a range covers is a valid pair, but what is kept differs from
 * gs_bin_tiles_bounded: the block entries past the capacity (the deepest
 * pairs') are dropped first, then the tiles' lists are cut at the capacity
 * in tile order (the tile that crosses it keeps its shallowest records,
 * later tiles keep none). No counterpart in the reference. */
int gs_bin_blocks_tiles_bounded(const int32_t* order, const int64_t* starts,
                                const int32_t* rects, int64_t count, int64_t capacity,
                                const int64_t* totals, int64_t images, int32_t width,
                                int32_t height, int32_t* point_list, int32_t* ranges,
                                uint32_t* overflow, void* workspace, size_t workspace_bytes,
                                void* stream);

/* ------------------------------------------------------------------ */
/* Kernels 4 and 5: tile compositors (renderForward / renderBackward,
 * rasterize.cu:230-399). neural = 0 selects the four-frequency Gabor
 * appearance (18 floats per row), 1 the per-surfel SIREN (57 floats).     */

/* Scratch bytes for gs_render_forward / gs_render_backward: the tile
 * dispatch order (heaviest tiles first) and per-tile contributor maxima. */
size_t gs_render_workspace_size(int64_t images, int32_t width, int32_t height);
/* Workspace of gs_render_backward: the forward's plus the order of the split
 * tiles' segments. */
size_t gs_render_backward_workspace_size(int64_t images, int32_t width, int32_t height,
                                         int64_t segment_capacity);

/* Map outputs and map gradients are passed as five channel groups in map
 * order - rgb (channels 0-2), alpha (3), depth (4), normals (5-7),
 * distortion (8) - as a host array of GS_MAP_GROUPS device pointers plus a
 * host array of 2*GS_MAP_GROUPS element strides (pixel stride, channel
 * stride per group): channel k of group g at pixel p is
 * data[g][p * strides[2g] + k * strides[2g+1]], p = (image*H + y)*W + x.
 * One [I,H,W,9] tensor is data[g] = maps + first channel of g with strides
 * (9, 1); separate [I,H,W,k] tensors and strided gradient views of a
 * caller's loss are passed the same way, without copies. */
#define GS_MAP_GROUPS 5

/* Replay lists (an addition; the reference has none): when replay and
 * replay_counts are non-null, the forward also writes, for every tile, the
 * point-list entries that at least one of its pixels composited, in list
 * order, into replay [replay_capacity, 2] int32 at the tile's range start:
 * {pair index, position in the tile's list | quadrant bits << 28}, where
 * bit 28 + q is set when a pixel of 8x8 quadrant q (q = 2 * (y >= 8) +
 * (x >= 8) within the tile) took the record; replay_counts [I*tw*th] int32
 * receives each list's length. replay_capacity is the point list's length
 * and must be below 2^28. Null pointers skip them. */
int gs_render_forward(int32_t neural, const float* geometry, const float* appearance,
                      const float* opacities, const int64_t* primitive_ids,
                      const float* backgrounds, const int32_t* point_list,
                      const int32_t* ranges, int64_t images, int32_t width, int32_t height,
                      float near_plane, float far_plane, float* const* maps,
                      const int64_t* map_strides, float* state, int32_t* contributors,
                      int32_t* replay, int64_t replay_capacity, int32_t* replay_counts,
                      int32_t segment_length, float* segment_state, int32_t* segment_index,
                      int64_t segment_capacity, void* workspace, size_t workspace_bytes,
                      void* stream);

/* Split tiles (segment_length > 0, a multiple of 64; 0 turns it off and
 * the three buffers are ignored; the backward needs the replay lists). No counterpart
 * in the reference, which walks each tile in one thread block. A tile whose
 * point list is longer than segment_length records is split into
 * K = ceil(length / segment_length) segments with K checkpoint slots,
 * assigned in tile order. The forward walks every segment in its own
 * workgroup, with the transmittance in front of it taken as 1, and a
 * second kernel merges the segments per pixel in list order, in closed
 * form, or by walking a segment again with the true transmittance where
 * the 1e-4 stop rule falls inside it. The backward then replays each
 * segment in its own workgroup from its checkpoint.
 * segment_state [segment_capacity][13][256] float32 receives each
 * checkpoint's per-pixel prefix state after every segment (transmittance,
 * rgb, depth, normals and the two depth moments; the last slot of a tile
 * holds its final state); segment_index int32 of length
 * E + 2 * (I*tw*th + segment_capacity), E = I*tw*th + segment_capacity
 * rounded up to even, receives each tile's first slot (-1: not split), then
 * per slot the replay-list length at its checkpoint, then (from int E) the
 * forward's work list. Slots past segment_capacity are not used (their
 * tiles are not split); floor(M / L) + min(I*tw*th, floor(M / (L + 1))) + 1
 * slots always suffice (M = point-list length, L = segment_length: a tile of
 * n > L records takes ceil(n / L) <= floor(n / L) + 1 slots, and at most
 * M / (L + 1) tiles are that long). gs_render_backward takes the same
 * arguments. */

/* gs_render_forward without a workspace argument. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation). The forward's only scratch, the tiles' dispatch order, lives
 * in a static device array of GS_RENDER_STATIC_MAX_TILES ints (4 MiB per
 * GPU, held until the process ends); more image tiles than that return
 * GS_ERR_WORKSPACE before any launch. Nothing is allocated. Every call on a
 * GPU shares that GPU's array, so calls that overlap on one GPU (on
 * different streams or threads) race; each call rewrites the order of all
 * its tiles before reading it, so nothing has to be cleared between calls.
 * Outputs are identical to gs_render_forward's (without split tiles). */
#define GS_RENDER_STATIC_MAX_TILES (1 << 20)
int gs_render_forward_static(int32_t neural, const float* geometry, const float* appearance,
                             const float* opacities, const int64_t* primitive_ids,
                             const float* backgrounds, const int32_t* point_list,
                             const int32_t* ranges, int64_t images, int32_t width,
                             int32_t height, float near_plane, float far_plane,
                             float* const* maps, const int64_t* map_strides, float* state,
                             int32_t* contributors, int32_t* replay, int64_t replay_capacity,
                             int32_t* replay_counts, void* stream);

/* Gradients are ACCUMULATED (global float atomics) into grad_geometry
 * [Q,17], grad_appearance [P,A], grad_opacities [P], grad_backgrounds
 * [I,3]; the caller zero-initialises them. grad_appearance_columns (an
 * addition; null for grad_appearance): for the neural renderer, a host
 * array of four device pointers that receive the appearance gradient as the
 * SIREN's parameter groups instead - input weights [P,30], input biases
 * [P,6], output weights [P,18], output biases [P,3] (appearance columns
 * 0-29, 30-35, 36-53, 54-56; null only when P is 0) - so that a caller
 * whose parameters are those four tensors, concatenated into the
 * appearance rows for the forward, needs no copies of the gradient slices
 * (the reference's caller takes them through autograd,
 * rendering.py:349-356). grad_maps uses the channel-group
 * form above; a null group pointer means a zero gradient for that group.
 * replay / replay_counts: the forward's replay lists, or both null; with
 * them the backward replays only the records some pixel took (the same
 * gradients: the other records contribute exact zeros). segment_*: the
 * forward's split-tile arguments (segment_length 0: none). The workspace is
 * gs_render_backward_workspace_size(images, width, height, segment_capacity)
 * bytes (segment_capacity 0 without split tiles). */
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
                       void* stream);

/* ------------------------------------------------------------------ */
/* Diagnostics. No counterpart in the reference. The same sources built with
 * -DGS_DIAGNOSTICS form libgabor_hip_diag.so, whose compositors also record
 * (a) per tile, the wall-clock stamps at which its workgroup began and ended,
 * in forward_span / backward_span [tiles][2] (int64, wall-clock ticks), and
 * (b) per (record, wave) the backward processes, the number of the wave's 64
 * lanes that take the record, as a histogram added into lanes [65] (uint64;
 * the caller clears it), and (c) work counters added into counters [8]
 * (uint64; the caller clears it): [0] the forward's (pixel, record) visits
 * of in-image pixels, every list record up to the one that stops the pixel
 * or to the end of its list (a split tile's segments count their relative
 * walks); [1] the (record, wave) pairs the forward processed, times 64
 * lanes; [2] the (record, wave) pairs the backward processed; the wave
 * steps those would take if each 32-lane half (8x4 pixels) or each 16-lane
 * block (4x4) of the wave's quadrant walked its own records: [3] halves and
 * [4] blocks at best (per batch the largest number of records any half or
 * block takes), [5] halves and [6] blocks in list order (records taken by
 * one half or block packed between records taken by several); [7] unused.
 * These cost a few instructions per processed (record, wave), so the
 * diagnostics library is for measurement only.                          */

/* *available = 1 in the diagnostics library, 0 in the product library;
 * *wall_clock_khz = the current device's wall-clock rate. */
int gs_diagnostics_query(int32_t* available, int32_t* wall_clock_khz);

/* Set the diagnostics targets on the current device (device pointers, null
 * to record nothing; spans are written for tile indices below `tiles`).
 * Synchronous. The product library returns GS_ERR_ARGUMENT. */
int gs_diagnostics_set(unsigned long long* lanes, long long* forward_span,
                       long long* backward_span, int64_t tiles, unsigned long long* counters);

/* ------------------------------------------------------------------ */
/* Kernel timing for measurement: when enabled, each compositor / sort /
 * projection launch is bracketed by HIP events on its own stream.        */

/* Kernel families reported by gs_profile_read. */
#define GS_PROF_PROJECT_FWD 0
#define GS_PROF_PROJECT_BWD 1
#define GS_PROF_SH_FWD 2
#define GS_PROF_SH_BWD 3
#define GS_PROF_BINNING 4
#define GS_PROF_SORT 5
#define GS_PROF_RENDER_FWD 6
#define GS_PROF_RENDER_BWD 7
#define GS_PROF_VALIDATE 8
#define GS_PROF_COUNT 9

/* Enable (1) or disable (0) event timing; enabling clears the totals. */
int gs_profile_enable(int32_t enable);

/* Synchronise pending events and report total milliseconds and launch
 * count of one kernel family since the last enable. */
int gs_profile_read(int32_t family, double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif

#endif /* GABOR_HIP_H */
