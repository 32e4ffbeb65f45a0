"""Public surface renderers and explicit tensor contracts (MI355X HIP backend).

Drop-in counterpart of the reference's ``src/gabor_splatting/rendering.py``:
the same public functions, keyword options and defaults, error types and
messages, ``[..., C, H, W, ch]`` outputs and ``meta`` dict. Projection, SH,
packing, binning, sorting and both compositors run as hand-written gfx950
HIP kernels (``libgabor_hip.so``, bound in ``_native``); PyTorch only
allocates memory, provides the stream and joins the autograd graph.
"""

from __future__ import annotations

import functools
import math
from typing import Any

import torch
from torch.autograd.function import once_differentiable

from . import _native


_SIDE_STREAMS: dict[int, torch.cuda.Stream] = {}
# Whether the neural renderer hands Composite the SIREN's four parameter
# groups, whose gradients the backward kernel then writes in place (True),
# or their concatenation into [S*N, 57] rows, as the reference does, whose
# gradient autograd slices and copies into the groups (False); the results
# are the same.
_NEURAL_COLUMNS = True
# Accumulator elements from which the backward's zero fill runs on a side
# stream (16 MB).
_SIDE_FILL_MIN = 1 << 22


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """A second stream of the device (default priority) for work that only
    has to finish before the backward: the accumulators' zero fill."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    stream = _SIDE_STREAMS.get(index)
    if stream is None:
        stream = _SIDE_STREAMS[index] = torch.cuda.Stream(device=device)
    return stream


_ZERO_BACKGROUNDS: dict[tuple, torch.Tensor] = {}


def _zero_backgrounds(device: torch.device, shape: tuple) -> torch.Tensor:
    """The default backgrounds, zeros of `shape` (rendering.py:295-296 makes
    them each call): kept per device and shape, since the renderers only
    read them and no caller receives them, so a step launches no fill for
    them. A kept tensor is made outside inference mode (autograd saves it),
    and its fill has finished before it is first returned, so that every
    stream reads zeros; during a graph capture, where a fill would only be
    recorded, a fresh tensor is made instead, as the reference does."""
    if torch.cuda.is_current_stream_capturing():
        return torch.zeros(shape, dtype=torch.float32, device=device)
    key = (device, shape)
    zeros = _ZERO_BACKGROUNDS.get(key)
    if zeros is None:
        if len(_ZERO_BACKGROUNDS) >= 64:
            _ZERO_BACKGROUNDS.clear()
        with torch.inference_mode(False):
            zeros = torch.zeros(shape, dtype=torch.float32, device=device)
        torch.cuda.current_stream(device).synchronize()
        _ZERO_BACKGROUNDS[key] = zeros
    return zeros


def _shaped(tensor: torch.Tensor, shape: tuple) -> torch.Tensor:
    """``tensor`` itself when it already has ``shape`` (no view node joins the
    autograd graph), else its reshape."""
    return tensor if tuple(tensor.shape) == shape else tensor.reshape(shape)


class Composite(torch.autograd.Function):
    """Tile compositor with first-order reverse mode (rendering.py:14-71).

    ``projected_means`` holds the same values as the geometry rows' xy
    columns; it is an input only so that the compositor's screen-filter
    gradient (gg[:, 9:11]) reaches it as an autograd node, as in the
    reference where ``meta["projected_means"]`` feeds the geometry.

    The nine map channels come out as five tensors - rgb, alpha, depth,
    normals, distortion, each [..., C, H, W, k] - rather than as slices of one
    [I,H,W,9] tensor: autograd would scatter the gradient of every slice
    into its own zero-filled full-size tensor and sum the five, while here
    the backward kernel reads each group's gradient where it lies (for a
    loss over ``torch.cat`` of the maps, straight out of the concatenated
    gradient) and missing groups cost nothing. With ``single`` (the
    single_map_storage context) it returns the reference's one [..., C, H,
    W, 9] tensor, which render() slices as the reference does.
    """

    @staticmethod
    def forward(
        ctx: Any, geometry, projected_means, appearance, opacities, primitive_ids, image_ids,
        radii, backgrounds, width, height, neural, near_plane, far_plane, bounded=None,
        grad_mode=True, violations=None, single=False, input_biases=None,
        output_weights=None, output_biases=None,
    ):
        # backgrounds [..., C, 3]; the maps come out as [..., C, H, W, k]
        # directly (the kernels see them as [I, H, W, k]), so the caller's
        # shapes need no view nodes in the autograd graph. With `single`
        # they come out as one [..., C, H, W, 9] tensor instead (the
        # reference's layout, rendering.py:375-400), which the kernels write
        # through five strided channel groups.
        image_shape = tuple(backgrounds.shape[:-1]) + (height, width)
        ctx.background_shape = backgrounds.shape
        ctx.single = single
        backgrounds = backgrounds.reshape(-1, 3)
        images = backgrounds.size(0)
        if single:
            shaped = torch.empty(image_shape + (sum(_native.MAP_GROUPS),), dtype=torch.float32,
                                 device=geometry.device)
            outputs = _native.split_map_groups(shaped.view(images, height, width, -1))
        else:
            shaped = tuple(
                torch.empty(image_shape + (k,), dtype=torch.float32, device=geometry.device)
                for k in _native.MAP_GROUPS
            )
            outputs = tuple(t.view(images, height, width, t.shape[-1]) for t in shaped)
        # The backward's zeroed accumulators are cleared while the host waits
        # for the intersection count. Without a capacity, a large fill (one
        # write of every accumulator, HBM-bound) goes to a side stream, where
        # it runs beside the latency-bound binning kernels, or beside the
        # previous step's compositors, instead of between them; the
        # backward's stream waits for it (config 4: 2.380 -> 2.371 ms per
        # step). A small one stays on the render's stream, where it costs
        # less host time than the stream switch (config 0: 0.623 -> 0.569
        # ms). With a capacity (renders a caller may capture in a graph) it
        # stays on the render's stream too: forked into a captured graph, the
        # fill made replays slower (configs 0-2 by 2-17%), not faster.
        ctx.accumulators = None
        ctx.accumulator_stream = None
        # The neural appearance may come as the SIREN's four parameter groups
        # (appearance = the input weights). The compositors read it as the
        # concatenated [P, 57] rows (one contiguous gather per record), made
        # here, and the backward writes its gradient straight into the four
        # groups' accumulators, which autograd hands to the parameters
        # without the slice copies a concatenation's backward makes.
        ctx.columns = input_biases is not None
        groups = (appearance, input_biases, output_weights, output_biases)
        rows = torch.cat(groups, dim=1) if ctx.columns else appearance
        like = groups if ctx.columns else appearance
        fill = geometry.numel() + rows.numel() + opacities.numel() + backgrounds.numel()

        def clear_accumulators():
            if bounded is None and fill >= _SIDE_FILL_MIN:
                side = _side_stream(geometry.device)
                with torch.cuda.stream(side):
                    ctx.accumulators = _native.zero_accumulators(geometry, like, opacities,
                                                                 backgrounds)
                ctx.accumulator_stream = side
            else:
                ctx.accumulators = _native.zero_accumulators(geometry, like, opacities,
                                                             backgrounds)

        # A backward can follow only when the caller records gradients (the
        # forward itself always runs without): only then are the backward's
        # accumulators and the replay lists prepared.
        needs_grad = grad_mode and any(ctx.needs_input_grad)
        overlap = clear_accumulators if needs_grad else None
        _, points, ranges, state, contributors, *replay = _native.rasterize_forward(
            geometry, rows, opacities, primitive_ids, image_ids, radii, backgrounds,
            width, height, neural, near_plane, far_plane, outputs=outputs, overlap=overlap,
            capacity=None if bounded is None else bounded.max_intersections,
            flags=None if bounded is None else bounded.record_binning, replay=needs_grad,
            violations=violations,
        )
        replay = replay[0] if replay else None
        # Binning and early termination are discrete: only the saved sorted
        # lists, per-pixel state, the tiles' replay lists (the records some
        # pixel took) and the split tiles' checkpoints are needed to replay
        # the tiles backwards.
        lists, counts, segments = replay if replay is not None else (None, None, None)
        length, checkpoints, checkpoint_index = segments if segments else (0, None, None)
        ctx.save_for_backward(
            geometry, rows, opacities, primitive_ids, backgrounds, points, ranges, state,
            contributors, lists, counts, checkpoints, checkpoint_index,
        )
        ctx.split = length
        ctx.options = (width, height, neural, near_plane, far_plane)
        ctx.set_materialize_grads(False)
        return shaped

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, *grad_groups):
        # A second backward through a retained graph gets fresh accumulators.
        accumulators, ctx.accumulators = ctx.accumulators, None
        if accumulators is not None and ctx.accumulator_stream is not None:
            # Filled on the side stream: wait for the fill, and keep the
            # memory from being reused before this stream is done with it.
            stream = torch.cuda.current_stream(accumulators[0].device)
            stream.wait_stream(ctx.accumulator_stream)
            for accumulator in accumulators:
                for tensor in (accumulator if isinstance(accumulator, tuple) else (accumulator,)):
                    tensor.record_stream(stream)
            ctx.accumulator_stream = None
        *saved, lists, counts, checkpoints, checkpoint_index = ctx.saved_tensors
        segments = (ctx.split, checkpoints, checkpoint_index) if ctx.split else None
        width, height = ctx.options[:2]
        if ctx.single:
            grad = grad_groups[0]
            if grad is None:
                groups = [None] * len(_native.MAP_GROUPS)
            else:
                grad = grad.reshape(-1, height, width, grad.shape[-1]).contiguous()
                groups = list(_native.split_map_groups(grad))
        else:
            groups = [None if g is None else g.reshape(-1, height, width, g.shape[-1])
                      for g in grad_groups]
        gg, ga, go, gb = _native.rasterize_backward(
            *saved, groups, *ctx.options, accumulators=accumulators,
            replay=None if lists is None else (lists, counts, segments),
        )
        column_grads = (None, None, None)
        if ctx.columns:
            # Without the forward's accumulators (a second backward through a
            # retained graph) the kernel wrote [P, 57] rows.
            ga, *column_grads = ga if isinstance(ga, tuple) else ga.split([30, 6, 18, 3], 1)
        return (gg, gg[:, 9:11], ga, go, None, None, None, gb.view(ctx.background_shape), None,
                None, None, None, None, None, None, None, None, *column_grads)


class ProjectRecords(torch.autograd.Function):
    """Projection, SH and compositor-record assembly as one HIP node.

    Replaces the reference's chain of PyTorch ops between its inputs and
    Composite (rendering.py:323-374): project_surfaces, SHColors, the
    per-camera expansion of shared appearance/opacity, the packing gathers
    and the geometry concatenation. Outputs: geometry rows [Q,17], projected
    means [Q,2], (with SH: appearance rows [Q,18], opacity rows [Q]), radii
    rows [Q], primitive ids [Q], image ids [Q], dense radii [S,C,N] and each
    row's scene, camera and surfel index [Q] (the meta ids of
    rendering.py:389-392).
    """

    @staticmethod
    def forward(ctx: Any, means, quaternions, scales, opacities, view_matrices, intrinsics,
                first, second, weights, magnitudes, phases, sh_degree, width, height,
                near_plane, far_plane, packed, fixed_rows=False):
        sh = None if sh_degree is None else (first, second)
        shared = None if sh_degree is None else (weights, magnitudes, phases)
        out = _native.records_forward(
            means, quaternions, scales, opacities, view_matrices, intrinsics, sh, shared,
            sh_degree, width, height, near_plane, far_plane, packed, fixed_rows,
        )
        row_of_pair = out["row_of_pair"]
        ctx.save_for_backward(means, quaternions, scales, view_matrices, intrinsics, first,
                              second, out["geometry"], row_of_pair)
        ctx.sh_degree = sh_degree
        ctx.set_materialize_grads(False)
        discrete = (out["row_radii"], out["primitive_ids"], out["image_ids"],
                    out["dense_radii"], out["scene_ids"], out["camera_ids"], out["surfel_ids"])
        ctx.mark_non_differentiable(*discrete)
        if sh_degree is None:
            return (out["geometry"], out["projected_means"], *discrete)
        return (out["geometry"], out["projected_means"], out["appearance"],
                out["opacity_rows"], *discrete)

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, g_geometry, g_projected, *rest):
        means, quats, scales, views, intrinsics, first, second, geometry, rows = ctx.saved_tensors
        sh_degree = ctx.sh_degree
        g_appearance, g_opacity = (rest[0], rest[1]) if sh_degree is not None else (None, None)
        if all(g is None for g in (g_geometry, g_projected, g_appearance, g_opacity)):
            return (None,) * 18
        grads = _native.records_backward(
            means, quats, scales, views, intrinsics,
            None if sh_degree is None else (first, second), sh_degree, rows, geometry,
            g_geometry, g_projected, g_appearance, g_opacity,
            camera_grads=ctx.needs_input_grad[4] or ctx.needs_input_grad[5],
        )
        g_means, g_quats, g_scales, g_views, g_intrinsics = grads[:5]
        g_first, g_second, g_weights, g_magnitudes, g_phases, g_opacities = grads[5:]
        return (g_means, g_quats, g_scales, g_opacities, g_views, g_intrinsics, g_first,
                g_second, g_weights, g_magnitudes, g_phases) + (None,) * 7


class ProjectSurfaces(torch.autograd.Function):
    """HIP projection of every (scene, camera, surfel) pair and its adjoint.

    Replaces the PyTorch ops of project_surfaces (rendering.py:176-218) and
    the autograd graph PyTorch builds through them.
    """

    @staticmethod
    def forward(ctx: Any, means, quaternions, scales, view_matrices, intrinsics, width,
                height, near_plane, far_plane):
        transform, xy, normals, directions, radii = _native.project_forward(
            means, quaternions, scales, view_matrices, intrinsics, width, height, near_plane,
            far_plane,
        )
        ctx.save_for_backward(means, quaternions, scales, view_matrices, intrinsics)
        ctx.mark_non_differentiable(radii)
        ctx.set_materialize_grads(False)
        return transform, xy, normals, directions, radii

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, g_transform, g_xy, g_normals, g_directions, _g_radii):
        if all(g is None for g in (g_transform, g_xy, g_normals, g_directions)):
            return (None,) * 9
        grads = _native.project_backward(
            *ctx.saved_tensors, g_transform, g_xy, g_normals, g_directions
        )
        return (*grads, None, None, None, None)


class SHColors(torch.autograd.Function):
    """Both classic SH colours from one direction per pair (rendering.py:221-238)."""

    @staticmethod
    def forward(ctx: Any, first, second, directions, degree):
        ctx.save_for_backward(first, second, directions)
        ctx.degree = degree
        return _native.evaluate_sh_forward(first, second, directions, degree)

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, grad_colors):
        gradients = _native.evaluate_sh_backward(
            *ctx.saved_tensors, grad_colors.contiguous(), ctx.degree
        )
        return *gradients, None


def check_tensor(
    name: str, value: torch.Tensor, shape: tuple[int, ...], device: torch.device
) -> None:
    """Require a contiguous float32 GPU tensor of an exact shape on `device`:
    TypeError for a non-tensor, ValueError for a wrong dtype or device, shape
    or layout (the C++ host checks every renderer input this way)."""
    _native.check_tensors({name: (value, shape)}, device)


# Value contracts in the order the reference lists them (rendering.py:95-148),
# one bit each above the per-tensor finiteness bits of gs_check_values.
VALUE_CONTRACTS = (
    "scales must be strictly positive",
    "opacities must lie in [0, 1]",
    "quaternions must be unit wxyz vectors",
    "view_matrices must have last row [0, 0, 0, 1]",
    "intrinsics must have last row [0, 0, 1]",
    "intrinsics fx and fy must be positive",
    "view_matrices rotations must be orthonormal",
    "view_matrices rotations must have determinant +1",
    "frequency_weights must be nonnegative",
    "frequency_magnitudes must be nonnegative",
    "frequency_weights must sum to one",
)


def describe_violations(names, violations: int) -> list[str]:
    """Messages of the contracts set in a gs_check_values word, in order."""
    messages = [
        f"{name} must contain only finite values"
        for bit, name in enumerate(names)
        if violations >> bit & 1
    ]
    first = _native.CHECK_MAX_TENSORS
    messages += [text for k, text in enumerate(VALUE_CONTRACTS) if violations >> (first + k) & 1]
    return messages


@torch.no_grad()
def check_values(
    tensors, quaternions, scales, opacities, view_matrices, intrinsics, appearance, neural
):
    """Numerical contracts, evaluated by one HIP kernel and read back once.

    Every tensor in ``tensors`` must be finite; scales positive; opacities
    in [0, 1]; quaternions unit; views rigid with last row [0, 0, 0, 1];
    intrinsics with last row [0, 0, 1] and positive focal lengths; classic
    frequency weights nonnegative and summing to one and magnitudes
    nonnegative. Raises ValueError naming every violated contract
    (rendering.py:88-153).
    """
    weights, magnitudes = (None, None) if neural else (appearance[2], appearance[3])
    violations = _native.check_values(
        [value for value, _ in tensors.values()], quaternions, scales, opacities,
        view_matrices, intrinsics, weights, magnitudes,
    )
    _raise_violations(list(tensors), violations)


def _raise_violations(names, violations: int) -> None:
    """ValueError naming every contract set in a gs_check_values word."""
    messages = describe_violations(names, violations & 0xFFFFFFFF)
    if messages:
        raise ValueError("; ".join(messages))


_check_values_on_device = check_values


class FixedCapacity:
    """Rendering without host synchronisation, for HIP graph capture.

    The reference reads the tile-intersection count on the host to size its
    point list (rasterize.cu:466-469) and reads the value checks' verdict
    back (rendering.py:149); neither can happen inside a captured graph, and
    both stall the host. While this context is active (``with
    fixed_capacity(max_intersections) as capacity:``), renders:

    * bin into a point list of ``max_intersections`` entries, the count
      staying on the device; if it exceeds the capacity, records are dropped
      (the deepest pairs' first, then the tile lists past the capacity in
      tile order; the tile sort, where the block path does not fit, drops
      the deepest records of the affected tiles) and a device flag is raised;
    * run the value checks (``validate=True``) on the device and keep the
      verdict instead of raising;
    * with ``packed=True``, keep one packed row per (scene, camera, surfel)
      pair instead of reading the visible count V back: ``meta["radii"]``,
      ``projected_means`` and the id tensors hold the V packed rows first,
      then rows of radius 0, projected mean 0 and id -1.

    ``check()``, called outside any capture, waits for the device and raises
    ValueError (violated value contracts, as ``check_values`` would) or
    RuntimeError (capacity exceeded, or binning found an index out of
    range); otherwise it returns the largest intersection count (0 if
    none), a guide for sizing the capacity. It reports everything rendered
    since the previous check, then starts afresh.

    The verdicts live in one small device tensor per GPU, allocated (and
    zeroed) outside any capture - when the context is created, or on first
    use on another device. Each render, eager or captured, folds its
    violation word, overflow flag and intersection count into it with
    device operations, so a captured graph folds them again on every
    replay: a check made right after capturing reads zeros (nothing ran
    yet), one made after replays reports those replays.
    """

    # Status words per device (int64): overflow flags OR-ed, largest
    # intersection count, then one OR-ed violation word per distinct list of
    # checked tensor names (classic and neural renders name them differently).
    _OVERFLOW, _PEAK, _FIRST_SLOT = 0, 1, 2
    _SLOTS = 6

    def __init__(self, max_intersections: int):
        if type(max_intersections) is not int or not 0 < max_intersections <= _native.INT_MAX:
            raise ValueError("max_intersections must be a positive int32 integer")
        self.max_intersections = max_intersections
        self._status: dict[torch.device, torch.Tensor] = {}
        self._names: list[tuple[str, ...]] = []
        if torch.cuda.is_available() and not torch.cuda.is_current_stream_capturing():
            self._status_on(torch.device("cuda", torch.cuda.current_device()))

    def __enter__(self) -> "FixedCapacity":
        _FIXED_CAPACITY.append(self)
        return self

    def __exit__(self, *exc) -> None:
        _FIXED_CAPACITY.remove(self)

    def _status_on(self, device: torch.device) -> torch.Tensor:
        status = self._status.get(device)
        if status is None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    f"fixed_capacity has no status words on {device}: create the context (or "
                    "render once eagerly) on that device before capturing"
                )
            status = torch.zeros(self._FIRST_SLOT + self._SLOTS, dtype=torch.int64,
                                 device=device)
            self._status[device] = status
        return status

    def record_binning(self, overflow: torch.Tensor, total: torch.Tensor) -> None:
        """Fold one render's overflow flag (int32 [1]) and intersection count
        (int64 [1]) into the device status (device operations only)."""
        status = self._status_on(overflow.device)
        status[self._OVERFLOW:self._OVERFLOW + 1].bitwise_or_(overflow)
        peak = status[self._PEAK:self._PEAK + 1]
        torch.maximum(peak, total, out=peak)

    def record_violations(self, word: torch.Tensor, names) -> None:
        """Fold one render's gs_check_values word (int32 [1]) into the slot of
        its tensor names (device operation only)."""
        names = tuple(names)
        if names not in self._names:
            if len(self._names) == self._SLOTS:
                raise RuntimeError("fixed_capacity: too many distinct input layouts")
            self._names.append(names)
        slot = self._FIRST_SLOT + self._names.index(names)
        self._status_on(word.device)[slot:slot + 1].bitwise_or_(word)

    def check(self) -> int:
        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            raise RuntimeError("fixed_capacity.check() cannot run during graph capture")
        overflow, peak, words = 0, 0, [0] * self._SLOTS
        for device, status in self._status.items():
            # Renders and replays may be queued on any stream of the device:
            # wait for all of them, and let the clearing finish before any
            # later render on another stream folds in its flags.
            torch.cuda.synchronize(device)
            host = status.tolist()
            status.zero_()
            torch.cuda.synchronize(device)
            overflow |= host[self._OVERFLOW]
            peak = max(peak, host[self._PEAK])
            words = [w | h for w, h in zip(words, host[self._FIRST_SLOT:])]
        messages = []
        for names, word in zip(self._names, words):
            for message in describe_violations(names, word & 0xFFFFFFFF):
                if message not in messages:
                    messages.append(message)
        if messages:
            raise ValueError("; ".join(messages))
        if overflow & _native.BINNING_BAD_INDEX:
            raise RuntimeError("binning produced an index out of range; the affected tiles "
                               "were rendered from substitute records")
        if overflow:
            raise RuntimeError(
                f"tile intersections ({peak}) exceeded the fixed capacity of "
                f"{self.max_intersections}; the affected renders dropped records"
            )
        return peak


_FIXED_CAPACITY: list[FixedCapacity] = []


def fixed_capacity(max_intersections: int) -> FixedCapacity:
    """Context manager: render without host synchronisation (see FixedCapacity)."""
    return FixedCapacity(max_intersections)


_SINGLE_MAP_STORAGE: list[bool] = []


class single_map_storage:  # noqa: N801 - a context manager, named like fixed_capacity
    """Context manager: renders inside it return rgb, alpha and the three map
    entries of ``meta`` as views of one [..., C, H, W, 9] tensor, as the
    reference does (rendering.py:375-400): same values, the reference's
    strides and shared ``_base``, and in-place changes of one view visible
    through the others. Outside it the five maps are separate contiguous
    tensors, which spares autograd from assembling the full [..., 9]
    gradient out of zero-filled slice gradients in the backward. Contexts
    nest; the setting is process-wide."""

    def __enter__(self) -> "single_map_storage":
        _SINGLE_MAP_STORAGE.append(True)
        return self

    def __exit__(self, *exc) -> None:
        _SINGLE_MAP_STORAGE.pop()


def quaternion_matrix(q: torch.Tensor) -> torch.Tensor:
    """Normalised wxyz quaternions to rotation matrices (rendering.py:156-173)."""
    q = q / torch.linalg.vector_norm(q, dim=-1, keepdim=True)
    w, x, y, z = q.unbind(-1)
    rows = (
        (1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)),
        (2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)),
        (2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)),
    )
    return torch.stack([torch.stack(row, -1) for row in rows], -2)


def project_surfaces(
    means, quaternions, scales, view_matrices, intrinsics, width, height, near_plane, far_plane
):
    """Projected planes T, conic centres, facing normals, world directions and radii."""
    return ProjectSurfaces.apply(
        means, quaternions, scales, view_matrices, intrinsics, width, height, near_plane,
        far_plane,
    )


_NEURAL_FIELDS = (
    ("input_weights", (6, 5)),
    ("input_biases", (6,)),
    ("output_weights", (3, 6)),
    ("output_biases", (3,)),
)


def render(
    means, quaternions, scales, opacities, appearance, view_matrices, intrinsics, width,
    height, backgrounds, packed, near_plane, far_plane, neural, sh_degree, validate,
    screen_points=None,
):
    """Validate, project every (scene, camera) pair, and composite in one launch.

    ``screen_points`` (optional, [Q, 2] float32, one row per projected pair)
    receives the gradient of the projected means, the screen-space gradient
    the upstream rasterizers write into their ``means2D`` argument; its
    values are not used."""
    if not isinstance(means, torch.Tensor) or means.ndim < 2 or means.shape[-1] != 3:
        raise ValueError("means must have shape [..., N, 3]")
    if not means.is_cuda or means.dtype != torch.float32:
        raise ValueError("means must be a CUDA float32 tensor")
    sizes_ok = type(width) is int and type(height) is int
    if not (sizes_ok and 0 < width < 2**30 and 0 < height < 2**30):
        raise ValueError("width and height must be positive integers smaller than 2**30")
    planes_ok = math.isfinite(near_plane) and math.isfinite(far_plane)
    if not (planes_ok and 0 < near_plane < far_plane):
        raise ValueError("clipping planes must be finite and satisfy 0 < near_plane < far_plane")
    if type(packed) is not bool:
        raise TypeError("packed must be bool")
    batch = tuple(means.shape[:-2])
    n = means.shape[-2]
    if not isinstance(view_matrices, torch.Tensor) or view_matrices.ndim != len(batch) + 3:
        raise ValueError("view_matrices must have shape [..., C, 4, 4]")
    cameras = view_matrices.shape[-3]
    scenes = math.prod(batch)
    if scenes < 1 or cameras < 1:
        raise ValueError("scene and camera dimensions must be nonempty")
    device = means.device
    if backgrounds is None:
        backgrounds = _zero_backgrounds(means.device, batch + (cameras, 3))
    tensors = {
        "means": (means, batch + (n, 3)),
        "quaternions": (quaternions, batch + (n, 4)),
        "scales": (scales, batch + (n, 2)),
        "opacities": (opacities, batch + (n,)),
        "view_matrices": (view_matrices, batch + (cameras, 4, 4)),
        "intrinsics": (intrinsics, batch + (cameras, 3, 3)),
        "backgrounds": (backgrounds, batch + (cameras, 3)),
    }
    if neural:
        fields = _NEURAL_FIELDS
    else:
        if sh_degree is not None and (type(sh_degree) is not int or not 0 <= sh_degree <= 3):
            raise ValueError("sh_degree must be None or an integer from 0 to 3")
        color = (3,) if sh_degree is None else ((sh_degree + 1) ** 2, 3)
        fields = (
            ("colors", color),
            ("secondary_colors", color),
            ("frequency_weights", (4,)),
            ("frequency_magnitudes", (4,)),
            ("phases", (4,)),
        )
    for (name, shape), value in zip(fields, appearance):
        tensors[name] = (value, batch + (n,) + shape)
    _native.check_tensors(tensors, device)
    if type(validate) is not bool:
        raise TypeError("validate must be bool")
    bounded = _FIXED_CAPACITY[-1] if _FIXED_CAPACITY else None
    violations = None
    if validate and bounded is None and check_values is not _check_values_on_device:
        # A caller's replacement of check_values runs where the reference calls it.
        check_values(
            tensors, quaternions, scales, opacities, view_matrices, intrinsics, appearance, neural
        )
    elif validate and bounded is None:
        # The verdict is read back with the intersection count, in the
        # forward's one synchronisation, and raised before anything is
        # composited: the same ValueError as check_values, one read-back less.
        weights, magnitudes = (None, None) if neural else (appearance[2], appearance[3])
        with torch.no_grad():
            word = _native.check_values_word(
                [value for value, _ in tensors.values()], quaternions, scales, opacities,
                view_matrices, intrinsics, weights, magnitudes,
            )
        violations = (word, functools.partial(_raise_violations, list(tensors)))
    elif validate:
        weights, magnitudes = (None, None) if neural else (appearance[2], appearance[3])
        with torch.no_grad():
            word = _native.check_values_word(
                [value for value, _ in tensors.values()], quaternions, scales, opacities,
                view_matrices, intrinsics, weights, magnitudes,
            )
            bounded.record_violations(word, list(tensors))

    views = _shaped(view_matrices, (scenes, cameras, 4, 4))
    cameras_k = _shaped(intrinsics, (scenes, cameras, 3, 3))
    columns = [None, None, None]  # the neural renderer's other SIREN groups
    if sh_degree is not None:
        # Camera-specific SH colours: appearance and opacity rows per pair,
        # written by the HIP record kernel.
        k = (sh_degree + 1) ** 2
        (geometry, projected_means, parameters, opacity_rows, row_radii, primitive_ids,
         image_ids, dense_radii, scene_ids, camera_ids, surfel_ids) = ProjectRecords.apply(
            _shaped(means, (scenes, n, 3)), _shaped(quaternions, (scenes, n, 4)),
            _shaped(scales, (scenes, n, 2)), _shaped(opacities, (scenes, n)), views, cameras_k,
            _shaped(appearance[0], (scenes, n, k, 3)), _shaped(appearance[1], (scenes, n, k, 3)),
            _shaped(appearance[2], (scenes, n, 4)), _shaped(appearance[3], (scenes, n, 4)),
            _shaped(appearance[4], (scenes, n, 4)), sh_degree, width, height, near_plane,
            far_plane, packed, bounded is not None,
        )
    else:
        # One appearance row per surfel, shared by every camera of its scene.
        (geometry, projected_means, row_radii, primitive_ids, image_ids, dense_radii,
         scene_ids, camera_ids, surfel_ids) = ProjectRecords.apply(
            _shaped(means, (scenes, n, 3)), _shaped(quaternions, (scenes, n, 4)),
            _shaped(scales, (scenes, n, 2)), None, views, cameras_k, None, None, None, None, None,
            None, width, height, near_plane, far_plane, packed, bounded is not None,
        )
        if neural and _NEURAL_COLUMNS:
            # The SIREN's four parameter groups as [S*N, w] views of the
            # caller's tensors: Composite concatenates them into the rows the
            # reference builds here (rendering.py:349-356) and writes their
            # gradients back group by group.
            parameters, *columns = (t.reshape(scenes * n, math.prod(shape))
                                    for t, (_, shape) in zip(appearance, fields))
        elif neural:
            flat = [t.reshape(scenes, n, math.prod(shape))
                    for t, (_, shape) in zip(appearance, fields)]
            parameters = torch.cat(flat, dim=-1).reshape(scenes * n, 57)
        else:
            flat = [t.reshape(scenes, n, math.prod(shape))
                    for t, (_, shape) in zip(appearance, fields)]
            parameters = torch.cat(flat, dim=-1).reshape(scenes * n, 18)
        opacity_rows = opacities.reshape(scenes * n)
    screen_means = projected_means
    if screen_points is not None:
        if screen_points.shape != projected_means.shape:
            raise ValueError(f"screen_points must have shape {tuple(projected_means.shape)}")
        screen_means = projected_means + (screen_points - screen_points.detach())
    single = bool(_SINGLE_MAP_STORAGE)
    maps = Composite.apply(
        geometry,
        screen_means,
        parameters,
        opacity_rows,
        primitive_ids,
        image_ids,
        row_radii,
        backgrounds,
        width,
        height,
        neural,
        near_plane,
        far_plane,
        bounded,
        torch.is_grad_enabled(),
        violations,
        single,
        *columns,
    )
    if single:  # views of one [..., C, H, W, 9] tensor (rendering.py:388-400)
        rgb, alpha, depth, normals, distortion = (
            maps[..., 0:3], maps[..., 3:4], maps[..., 4:5], maps[..., 5:8], maps[..., 8:9])
    else:
        rgb, alpha, depth, normals, distortion = maps
    meta = {
        "radii": row_radii if packed else dense_radii.reshape(batch + (cameras, n)),
        "projected_means": projected_means,
        "scene_ids": scene_ids,
        "camera_ids": camera_ids,
        "primitive_ids": surfel_ids,
        "packed": packed,
        "accumulated_depth": depth,
        "normals": normals,
        "distortion": distortion,
    }
    return rgb, alpha, meta


def rasterize_gabors(
    means: torch.Tensor,
    quaternions: torch.Tensor,
    scales: torch.Tensor,
    opacities: torch.Tensor,
    colors: torch.Tensor,
    secondary_colors: torch.Tensor,
    frequency_weights: torch.Tensor,
    frequency_magnitudes: torch.Tensor,
    phases: torch.Tensor,
    view_matrices: torch.Tensor,
    intrinsics: torch.Tensor,
    width: int,
    height: int,
    *,
    backgrounds: torch.Tensor | None = None,
    packed: bool = False,
    near_plane: float = 0.2,
    far_plane: float = 100.0,
    sh_degree: int | None = None,
    validate: bool = True,
) -> tuple[torch.Tensor, torch.Tensor, dict[str, Any]]:
    """Render four-frequency Gabor surfaces over scene and camera batches.

    Geometry: means [..., N, 3], unit wxyz quaternions [..., N, 4], positive
    tangent scales [..., N, 2], activated opacities [..., N]. Colours are
    [..., N, 3] or, with ``sh_degree``, SH coefficients [..., N, (d+1)**2, 3].
    Frequency weights (nonnegative, summing to one), magnitudes (cycles per
    scaled local unit) and phases (radians) are [..., N, 4]. Cameras are
    rigid world-to-camera [..., C, 4, 4] and pinhole [..., C, 3, 3]. All
    tensors are contiguous float32 on one GPU. Returns RGB [..., C, H, W, 3],
    alpha [..., C, H, W, 1] and metadata (rendering.py:403-456).
    """
    return render(
        means, quaternions, scales, opacities,
        (colors, secondary_colors, frequency_weights, frequency_magnitudes, phases),
        view_matrices, intrinsics, width, height, backgrounds, packed, near_plane, far_plane,
        False, sh_degree, validate,
    )


def rasterize_neural_gabors(
    means: torch.Tensor,
    quaternions: torch.Tensor,
    scales: torch.Tensor,
    opacities: torch.Tensor,
    input_weights: torch.Tensor,
    input_biases: torch.Tensor,
    output_weights: torch.Tensor,
    output_biases: torch.Tensor,
    view_matrices: torch.Tensor,
    intrinsics: torch.Tensor,
    width: int,
    height: int,
    *,
    backgrounds: torch.Tensor | None = None,
    packed: bool = False,
    near_plane: float = 0.2,
    far_plane: float = 100.0,
    validate: bool = True,
) -> tuple[torch.Tensor, torch.Tensor, dict[str, Any]]:
    """Render per-surfel 5->6->3 SIRENs (sine frequency 30, sigmoid RGB).

    Input weights/biases are [..., N, 6, 5] / [..., N, 6]; output weights/
    biases [..., N, 3, 6] / [..., N, 3]. The network input is (u/3, v/3)
    followed by the world direction camera -> centre (rendering.py:459-507).
    """
    return render(
        means, quaternions, scales, opacities,
        (input_weights, input_biases, output_weights, output_biases),
        view_matrices, intrinsics, width, height, backgrounds, packed, near_plane, far_plane,
        True, None, validate,
    )
