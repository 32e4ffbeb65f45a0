// Host side of the renderer's per-render calls, in C++: the counterpart of
// the reference's C++ host functions rasterizeForward / rasterizeBackward
// (rasterize.cu:402-529), extended to the fused projection front end and
// the depth-first binning of this library.
//
// Every function here keeps the signature, checks, messages and outputs of
// the Python host function of the same name in _native.py, which now only
// forwards to it; structural violations raise RuntimeError, as TORCH_CHECK
// does in the reference. Outputs come from the torch caching allocator and
// every launch goes to the current HIP stream of the tensors' device. A
// render crosses into C++ a handful of times instead of running a few
// hundred Python statements and ctypes conversions per call, which is most
// of a small render's time.
//
// The C ABI entry points are called through a table of function addresses
// that the Python module which loaded libgabor_hip.so hands over (bind), so
// that when it switches to another build of the same sources (the
// diagnostics library) these calls follow.

#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "gabor_hip.h"

namespace py = pybind11;

namespace {

constexpr int64_t kTile = 16;
constexpr int64_t kGeometry = 17;
constexpr int64_t kMapSize = 9;
constexpr int64_t kIntMax = 2147483647;
constexpr int64_t kReplayMaxEntries = (int64_t(1) << 28) - 1;
constexpr int64_t kCheckpointFloats = 13;
constexpr int kCheckMaxTensors = 16;
constexpr std::array<int64_t, 5> kMapGroups = {3, 1, 1, 3, 1};  // rgb, alpha, depth, normals, distortion

struct Api {
  decltype(&gs_last_error) last_error = nullptr;
  decltype(&gs_check_values) check_values = nullptr;
  decltype(&gs_scan_workspace_size) scan_workspace_size = nullptr;
  decltype(&gs_pack_visible) pack_visible = nullptr;
  decltype(&gs_records_forward) records_forward = nullptr;
  decltype(&gs_records_backward_workspace_size) records_backward_workspace_size = nullptr;
  decltype(&gs_records_backward) records_backward = nullptr;
  decltype(&gs_bin_order_workspace_size) bin_order_workspace_size = nullptr;
  decltype(&gs_bin_order_count) bin_order_count = nullptr;
  decltype(&gs_bin_order_sort) bin_order_sort = nullptr;
  decltype(&gs_bin_tiles_workspace_size) bin_tiles_workspace_size = nullptr;
  decltype(&gs_bin_tiles) bin_tiles = nullptr;
  decltype(&gs_bin_tiles_bounded) bin_tiles_bounded = nullptr;
  decltype(&gs_bin_blocks_tiles_bounded) bin_blocks_tiles_bounded = nullptr;
  decltype(&gs_bin_blocks_fit) bin_blocks_fit = nullptr;
  decltype(&gs_bin_blocks_count) bin_blocks_count = nullptr;
  decltype(&gs_bin_blocks_sort) bin_blocks_sort = nullptr;
  decltype(&gs_bin_blocks_tiles_workspace_size) bin_blocks_tiles_workspace_size = nullptr;
  decltype(&gs_bin_blocks_tiles) bin_blocks_tiles = nullptr;
  decltype(&gs_render_workspace_size) render_workspace_size = nullptr;
  decltype(&gs_render_backward_workspace_size) render_backward_workspace_size = nullptr;
  decltype(&gs_render_forward) render_forward = nullptr;
  decltype(&gs_render_backward) render_backward = nullptr;
};

Api api;
bool bound = false;

template <typename F>
void take(const py::dict& table, const char* name, F& slot) {
  if (!table.contains(name))
    throw std::runtime_error(std::string("the entry point table lacks ") + name);
  const auto address = table[name].cast<uintptr_t>();
  if (address == 0) throw std::runtime_error(std::string("null address for ") + name);
  slot = reinterpret_cast<F>(address);
}

// Entry point addresses by name (the library's exported symbols).
void bind(const py::dict& table) {
  Api next;
  take(table, "gs_last_error", next.last_error);
  take(table, "gs_check_values", next.check_values);
  take(table, "gs_scan_workspace_size", next.scan_workspace_size);
  take(table, "gs_pack_visible", next.pack_visible);
  take(table, "gs_records_forward", next.records_forward);
  take(table, "gs_records_backward_workspace_size", next.records_backward_workspace_size);
  take(table, "gs_records_backward", next.records_backward);
  take(table, "gs_bin_order_workspace_size", next.bin_order_workspace_size);
  take(table, "gs_bin_order_count", next.bin_order_count);
  take(table, "gs_bin_order_sort", next.bin_order_sort);
  take(table, "gs_bin_tiles_workspace_size", next.bin_tiles_workspace_size);
  take(table, "gs_bin_tiles", next.bin_tiles);
  take(table, "gs_bin_tiles_bounded", next.bin_tiles_bounded);
  take(table, "gs_bin_blocks_tiles_bounded", next.bin_blocks_tiles_bounded);
  take(table, "gs_bin_blocks_fit", next.bin_blocks_fit);
  take(table, "gs_bin_blocks_count", next.bin_blocks_count);
  take(table, "gs_bin_blocks_sort", next.bin_blocks_sort);
  take(table, "gs_bin_blocks_tiles_workspace_size", next.bin_blocks_tiles_workspace_size);
  take(table, "gs_bin_blocks_tiles", next.bin_blocks_tiles);
  take(table, "gs_render_workspace_size", next.render_workspace_size);
  take(table, "gs_render_backward_workspace_size", next.render_backward_workspace_size);
  take(table, "gs_render_forward", next.render_forward);
  take(table, "gs_render_backward", next.render_backward);
  api = next;
  bound = true;
}

std::vector<std::string> entry_points() {
  return {"gs_last_error", "gs_check_values", "gs_scan_workspace_size", "gs_pack_visible",
          "gs_records_forward", "gs_records_backward_workspace_size", "gs_records_backward",
          "gs_bin_order_workspace_size", "gs_bin_order_count", "gs_bin_order_sort",
          "gs_bin_tiles_workspace_size", "gs_bin_tiles", "gs_bin_tiles_bounded",
          "gs_bin_blocks_fit", "gs_bin_blocks_count", "gs_bin_blocks_sort",
          "gs_bin_blocks_tiles_workspace_size", "gs_bin_blocks_tiles",
          "gs_bin_blocks_tiles_bounded", "gs_render_workspace_size",
          "gs_render_backward_workspace_size", "gs_render_forward", "gs_render_backward"};
}

[[noreturn]] void fail(const std::string& message) { throw std::runtime_error(message); }

inline void require(bool ok, const char* message) {
  if (!ok) fail(message);
}

void check(int status) {
  if (status == 0) return;
  const char* message = api.last_error ? api.last_error() : nullptr;
  if (message && *message) fail(message);
  fail("gabor HIP call failed with status " + std::to_string(status));
}

void check_hip(hipError_t status, const char* what) {
  if (status != hipSuccess) fail(std::string(what) + " failed: " + hipGetErrorString(status));
}

void require_bound() {
  if (!bound) fail("the HIP library's entry points are not bound (_host.bind)");
}

inline void* stream_of(const at::Device& device) {
  return c10::hip::getCurrentHIPStream(device.index()).stream();
}

template <typename T>
inline T* ptr(const at::Tensor& t) {
  return t.defined() ? static_cast<T*>(t.data_ptr()) : nullptr;
}

template <typename T>
inline T* ptr(const std::optional<at::Tensor>& t) {
  return t ? ptr<T>(*t) : nullptr;
}

inline at::TensorOptions on(const at::Device& device, at::ScalarType type) {
  return at::TensorOptions().dtype(type).device(device);
}

at::Tensor workspace(size_t bytes, const at::Device& device) {
  return at::empty({std::max<int64_t>(int64_t(bytes), 1)}, on(device, at::kByte));
}

void check_float(const at::Tensor& value, const at::Tensor& geometry) {
  require(value.is_cuda() && value.scalar_type() == at::kFloat,
          "native rendering requires CUDA float32 tensors");
  require(value.device() == geometry.device() && value.is_contiguous(),
          "native buffers must be contiguous on the geometry device");
}

// checkBuffers (rasterize.cu:410-422).
void check_buffers(const at::Tensor& geometry, const at::Tensor& appearance,
                   const at::Tensor& opacities, const at::Tensor& primitive_ids,
                   const at::Tensor& backgrounds, bool neural) {
  for (const at::Tensor* value : {&geometry, &appearance, &opacities, &backgrounds})
    check_float(*value, geometry);
  require(geometry.dim() == 2 && geometry.size(1) == kGeometry, "invalid geometry shape");
  require(geometry.size(0) <= kIntMax, "too many projected primitives");
  require(appearance.dim() == 2 && appearance.size(1) == (neural ? 57 : 18),
          "invalid appearance shape");
  require(opacities.dim() == 1 && opacities.size(0) == appearance.size(0),
          "invalid opacity shape");
  require(backgrounds.dim() == 2 && backgrounds.size(1) == 3 && backgrounds.size(0) > 0,
          "invalid backgrounds");
  require(primitive_ids.device() == geometry.device() && primitive_ids.is_contiguous() &&
              primitive_ids.scalar_type() == at::kLong && primitive_ids.dim() == 1 &&
              primitive_ids.size(0) == geometry.size(0),
          "invalid primitive IDs");
}

inline int64_t tiles_across(int64_t extent) { return (extent + kTile - 1) / kTile; }

bool same_shape(const at::Tensor& t, std::initializer_list<int64_t> shape) {
  return t.sizes().equals(c10::IntArrayRef(shape.begin(), shape.size()));
}

// --------------------------------------------------------------------------
// Argument checks of the public renderers (rendering.py:260-318).

// Python's repr of a tuple of ints: "()", "(5,)", "(1, 2)".
std::string tuple_repr(c10::IntArrayRef shape) {
  std::string text = "(";
  for (size_t i = 0; i < shape.size(); ++i) {
    if (i) text += ", ";
    text += std::to_string(shape[i]);
  }
  return text + (shape.size() == 1 ? ",)" : ")");
}

// Every entry name -> (value, shape) must be a contiguous float32 tensor of
// exactly that shape on `device`; the first that is not raises TypeError
// (not a tensor) or ValueError, with the Python checks' messages.
void check_tensors(const py::dict& tensors, const py::object& device) {
  const at::Device expected = device.cast<at::Device>();
  for (const auto& item : tensors) {
    const std::string name = py::str(item.first);
    const py::tuple entry = item.second.cast<py::tuple>();
    const py::handle value = entry[0];
    if (!THPVariable_Check(value.ptr())) throw py::type_error(name + " must be a torch.Tensor");
    const at::Tensor& t = THPVariable_Unpack(value.ptr());
    if (!(t.is_cuda() && t.scalar_type() == at::kFloat && t.device() == expected))
      throw py::value_error(name + " must be float32 on " + std::string(py::str(device)));
    const std::vector<int64_t> shape = entry[1].cast<std::vector<int64_t>>();
    if (!t.sizes().equals(shape))
      throw py::value_error(name + " must have shape " + tuple_repr(shape) + ", got " +
                            tuple_repr(t.sizes()));
    if (!t.is_contiguous()) throw py::value_error(name + " must be contiguous");
  }
}

// --------------------------------------------------------------------------
// The pinned read-back of the binning totals (and a value-check word).

// Each host thread keeps one pinned buffer and one event per device: the
// host waits on the event before reading the buffer and returning, so a
// later call on the same thread may reuse both.
struct Readback {
  int64_t* host = nullptr;
  std::array<hipEvent_t, 64> events{};
};

Readback& readback() {
  thread_local Readback state;
  if (!state.host) {
    void* memory = nullptr;
    check_hip(hipHostMalloc(&memory, 64, hipHostMallocDefault), "hipHostMalloc");
    state.host = static_cast<int64_t*>(memory);
  }
  return state;
}

hipEvent_t readback_event(Readback& state, const at::Device& device) {
  const int index = device.index();
  if (index < 0 || index >= int(state.events.size())) fail("device index out of range");
  if (!state.events[index])
    check_hip(hipEventCreateWithFlags(&state.events[index], hipEventDisableTiming),
              "hipEventCreateWithFlags");
  return state.events[index];
}

// --------------------------------------------------------------------------
// Input value contracts.

at::Tensor check_values_word(const std::vector<at::Tensor>& tensors,
                             const at::Tensor& quaternions, const at::Tensor& scales,
                             const at::Tensor& opacities, const at::Tensor& view_matrices,
                             const at::Tensor& intrinsics,
                             const std::optional<at::Tensor>& weights,
                             const std::optional<at::Tensor>& magnitudes) {
  require_bound();
  require(int(tensors.size()) <= kCheckMaxTensors, "too many tensors to check");
  const int64_t surfels = quaternions.numel() / 4;
  const int64_t images = view_matrices.numel() / 16;
  for (const at::Tensor& value : tensors) check_float(value, quaternions);
  for (const at::Tensor* value : {&quaternions, &scales, &opacities, &view_matrices, &intrinsics})
    check_float(*value, quaternions);
  if (weights) check_float(*weights, quaternions);
  if (magnitudes) check_float(*magnitudes, quaternions);
  require(quaternions.numel() == 4 * surfels && scales.numel() == 2 * surfels &&
              opacities.numel() == surfels && (!weights || weights->numel() == 4 * surfels) &&
              (!magnitudes || magnitudes->numel() == 4 * surfels),
          "surfel tensors disagree in size");
  require(view_matrices.numel() == 16 * images && intrinsics.numel() == 9 * images,
          "camera tensors disagree in size");
  std::array<const float*, kCheckMaxTensors> pointers{};
  std::array<int64_t, kCheckMaxTensors> sizes{};
  for (size_t i = 0; i < tensors.size(); ++i) {
    pointers[i] = ptr<const float>(tensors[i]);
    sizes[i] = tensors[i].numel();
  }
  const at::Device device = quaternions.device();
  c10::DeviceGuard guard(device);
  at::Tensor violations = at::empty({1}, on(device, at::kInt));
  check(api.check_values(pointers.data(), sizes.data(), int32_t(tensors.size()),
                         ptr<const float>(quaternions), ptr<const float>(scales),
                         ptr<const float>(opacities), ptr<const float>(weights),
                         ptr<const float>(magnitudes), surfels, ptr<const float>(view_matrices),
                         ptr<const float>(intrinsics), images, ptr<uint32_t>(violations),
                         stream_of(device)));
  return violations;
}

// --------------------------------------------------------------------------
// Visible-pair packing.

py::object pack_visible(const at::Tensor& radii, bool with_rows, bool sync) {
  require_bound();
  const at::Tensor flat = radii.reshape(-1);
  const int64_t count = flat.numel();
  const at::Device device = radii.device();
  c10::DeviceGuard guard(device);
  at::Tensor selected = at::empty({std::max<int64_t>(count, 1)}, on(device, at::kLong));
  at::Tensor rows;
  if (with_rows) rows = at::empty({std::max<int64_t>(count, 1)}, on(device, at::kInt));
  at::Tensor total = at::empty({1}, on(device, at::kLong));
  at::Tensor space = workspace(api.scan_workspace_size(count), device);
  check(api.pack_visible(ptr<const int32_t>(flat), count, ptr<int64_t>(selected),
                         ptr<int32_t>(rows), ptr<int64_t>(total), space.data_ptr(),
                         size_t(space.numel()), stream_of(device)));
  if (!sync) {
    if (with_rows)
      return py::make_tuple(selected.slice(0, 0, count), rows.slice(0, 0, count), total);
    return py::make_tuple(selected.slice(0, 0, count), total);
  }
  selected = selected.slice(0, 0, total.item<int64_t>());
  if (with_rows) return py::make_tuple(selected, rows.slice(0, 0, count));
  return py::cast(selected);
}

// --------------------------------------------------------------------------
// Fused projection + SH + record assembly (the renderer's front end).

struct RecordOutputs {
  at::Tensor geometry, projected_means, row_radii, primitive_ids, image_ids, appearance,
      opacity_rows, scene_ids, camera_ids, surfel_ids;
};

py::dict records_forward(const at::Tensor& means, const at::Tensor& quaternions,
                         const at::Tensor& scales, const std::optional<at::Tensor>& opacities,
                         const at::Tensor& view_matrices, const at::Tensor& intrinsics,
                         const std::optional<std::tuple<at::Tensor, at::Tensor>>& sh,
                         const std::optional<std::tuple<at::Tensor, at::Tensor, at::Tensor>>& shared,
                         const std::optional<int64_t>& sh_degree, int64_t width, int64_t height,
                         double near_plane, double far_plane, bool packed, bool fixed_rows) {
  require_bound();
  const at::Device device = means.device();
  const int64_t scenes = means.size(0), n = means.size(1);
  const int64_t cameras = view_matrices.size(1);
  const int64_t pairs = scenes * cameras * n;
  at::Tensor first, second, weights, magnitudes, phases;
  if (sh) std::tie(first, second) = *sh;
  if (shared) std::tie(weights, magnitudes, phases) = *shared;
  const int32_t degree = sh_degree ? int32_t(*sh_degree) : -1;
  void* stream = stream_of(device);

  auto launch = [&](const at::Tensor& row_of_pair, const at::Tensor& dense_radii,
                    const RecordOutputs& out) {
    check(api.records_forward(
        ptr<const float>(means), ptr<const float>(quaternions), ptr<const float>(scales),
        ptr<const float>(opacities), ptr<const float>(view_matrices),
        ptr<const float>(intrinsics), ptr<const float>(first), ptr<const float>(second),
        ptr<const float>(weights), ptr<const float>(magnitudes), ptr<const float>(phases),
        degree, scenes, cameras, n, int32_t(width), int32_t(height), float(near_plane),
        float(far_plane), ptr<const int32_t>(row_of_pair), ptr<int32_t>(dense_radii),
        ptr<float>(out.geometry), ptr<float>(out.projected_means), ptr<int32_t>(out.row_radii),
        ptr<int64_t>(out.primitive_ids), ptr<int64_t>(out.image_ids), ptr<float>(out.appearance),
        ptr<float>(out.opacity_rows), ptr<int64_t>(out.scene_ids), ptr<int64_t>(out.camera_ids),
        ptr<int64_t>(out.surfel_ids), stream));
  };

  c10::DeviceGuard guard(device);
  at::Tensor dense_radii = at::empty({scenes, cameras, n}, on(device, at::kInt));
  at::Tensor row_of_pair, selected;
  const bool padded = packed && fixed_rows;
  int64_t rows = pairs;
  if (packed) {
    launch(at::Tensor(), dense_radii, RecordOutputs{});
    const py::tuple packing = pack_visible(dense_radii, true, !padded).cast<py::tuple>();
    selected = packing[0].cast<at::Tensor>();
    row_of_pair = packing[1].cast<at::Tensor>();
    rows = selected.numel();
  }
  // Padded rows past the visible count are never written by the record
  // kernel: they are filled here so that binning culls them and the meta
  // outputs stay defined.
  const auto f32 = on(device, at::kFloat);
  const auto i32 = on(device, at::kInt);
  const auto i64 = on(device, at::kLong);
  RecordOutputs out;
  out.geometry = at::empty({rows, kGeometry}, f32);
  out.projected_means = padded ? at::zeros({rows, 2}, f32) : at::empty({rows, 2}, f32);
  out.row_radii = padded ? at::zeros({rows}, i32) : at::empty({rows}, i32);
  out.primitive_ids = at::empty({rows}, i64);
  out.image_ids = at::empty({rows}, i64);
  if (degree >= 0) {
    out.appearance = at::empty({rows, 18}, f32);
    out.opacity_rows = at::empty({rows}, f32);
  }
  const at::Tensor meta_ids = padded ? at::full({3, rows}, -1, i64) : at::empty({3, rows}, i64);
  out.scene_ids = meta_ids.select(0, 0);
  out.camera_ids = meta_ids.select(0, 1);
  out.surfel_ids = meta_ids.select(0, 2);
  if (rows) launch(row_of_pair, packed ? at::Tensor() : dense_radii, out);

  auto maybe = [](const at::Tensor& t) -> py::object {
    return t.defined() ? py::cast(t) : py::none();
  };
  py::dict result;
  result["geometry"] = out.geometry;
  result["projected_means"] = out.projected_means;
  result["row_radii"] = out.row_radii;
  result["primitive_ids"] = out.primitive_ids;
  result["image_ids"] = out.image_ids;
  if (degree >= 0) {
    result["appearance"] = out.appearance;
    result["opacity_rows"] = out.opacity_rows;
  }
  result["scene_ids"] = out.scene_ids;
  result["camera_ids"] = out.camera_ids;
  result["surfel_ids"] = out.surfel_ids;
  result["dense_radii"] = dense_radii;
  result["row_of_pair"] = maybe(row_of_pair);
  result["selected"] = maybe(selected);
  return result;
}

at::Tensor contiguous_or_undefined(const std::optional<at::Tensor>& value) {
  return value ? value->contiguous() : at::Tensor();
}

py::tuple records_backward(const at::Tensor& means, const at::Tensor& quaternions,
                           const at::Tensor& scales, const at::Tensor& view_matrices,
                           const at::Tensor& intrinsics,
                           const std::optional<std::tuple<at::Tensor, at::Tensor>>& sh,
                           const std::optional<int64_t>& sh_degree,
                           const std::optional<at::Tensor>& row_of_pair,
                           const at::Tensor& geometry,
                           const std::optional<at::Tensor>& grad_geometry_in,
                           const std::optional<at::Tensor>& grad_projected_in,
                           const std::optional<at::Tensor>& grad_appearance_in,
                           const std::optional<at::Tensor>& grad_opacity_in,
                           bool camera_grads) {
  require_bound();
  const at::Device device = means.device();
  const int64_t scenes = means.size(0), n = means.size(1);
  const int64_t cameras = view_matrices.size(1);
  const int32_t degree = sh_degree ? int32_t(*sh_degree) : -1;
  at::Tensor first, second;
  if (sh) std::tie(first, second) = *sh;
  const at::Tensor grad_geometry = contiguous_or_undefined(grad_geometry_in);
  // The compositor's gradient of the projected means is the xy columns of
  // its geometry gradient; rows of any stride are read in place.
  at::Tensor grad_projected;
  if (grad_projected_in) {
    const at::Tensor& g = *grad_projected_in;
    grad_projected = (g.dim() == 2 && g.stride(1) == 1 && g.stride(0) >= 2) ? g : g.contiguous();
  }
  const int64_t projected_stride = grad_projected.defined() ? grad_projected.stride(0) : 2;
  at::Tensor grad_appearance = contiguous_or_undefined(grad_appearance_in);
  const at::Tensor grad_opacity = contiguous_or_undefined(grad_opacity_in);
  c10::DeviceGuard guard(device);
  const at::Tensor g_means = at::empty_like(means);
  const at::Tensor g_quats = at::empty_like(quaternions);
  const at::Tensor g_scales = at::empty_like(scales);
  // Without camera_grads the camera adjoint is skipped (null pointers) and
  // the camera gradients are returned as None.
  const at::Tensor g_views = camera_grads ? at::empty_like(view_matrices) : at::Tensor();
  const at::Tensor g_intrinsics = camera_grads ? at::empty_like(intrinsics) : at::Tensor();
  std::array<at::Tensor, 6> sh_grads;
  if (degree >= 0) {
    if (!grad_appearance.defined())
      grad_appearance = at::zeros({geometry.size(0), 18}, on(device, at::kFloat));
    const auto f32 = on(device, at::kFloat);
    sh_grads = {at::empty_like(first), at::empty_like(second), at::empty({scenes, n, 4}, f32),
                at::empty({scenes, n, 4}, f32), at::empty({scenes, n, 4}, f32),
                at::empty({scenes, n}, f32)};
  }
  const at::Tensor space =
      workspace(api.records_backward_workspace_size(scenes, cameras, n, degree), device);
  check(api.records_backward(
      ptr<const float>(means), ptr<const float>(quaternions), ptr<const float>(scales),
      ptr<const float>(view_matrices), ptr<const float>(intrinsics), ptr<const float>(first),
      ptr<const float>(second), degree, scenes, cameras, n, ptr<const int32_t>(row_of_pair),
      ptr<const float>(geometry), ptr<const float>(grad_geometry),
      ptr<const float>(grad_projected), projected_stride, ptr<const float>(grad_appearance),
      ptr<const float>(grad_opacity), ptr<float>(g_means), ptr<float>(g_quats),
      ptr<float>(g_scales), ptr<float>(g_views), ptr<float>(g_intrinsics),
      ptr<float>(sh_grads[0]), ptr<float>(sh_grads[1]), ptr<float>(sh_grads[2]),
      ptr<float>(sh_grads[3]), ptr<float>(sh_grads[4]), ptr<float>(sh_grads[5]),
      space.data_ptr(), size_t(space.numel()), stream_of(device)));
  py::tuple result(11);
  result[0] = g_means;
  result[1] = g_quats;
  result[2] = g_scales;
  result[3] = camera_grads ? py::cast(g_views) : py::none();
  result[4] = camera_grads ? py::cast(g_intrinsics) : py::none();
  for (int k = 0; k < 6; ++k)
    result[5 + k] = sh_grads[k].defined() ? py::cast(sh_grads[k]) : py::none();
  return result;
}

// --------------------------------------------------------------------------
// Depth-first binning.

// Stage 1 of depth-first binning in its two calls. count_stage makes the
// rectangles and counts and sums M and V into totals; sort_stage orders the
// pairs by depth from the same workspace.
struct OrderStage {
  at::Tensor order, starts, rects, totals, space;
  int64_t count = 0;
  bool blocks = false;               // block path (gs_bin_blocks_count)
  float near_plane = 0.f, far_plane = 0.f;  // its depth-key range; 0, 0: raw keys
};

OrderStage count_stage(const at::Tensor& geometry, const at::Tensor& radii,
                       const at::Tensor& image_ids, int64_t width, int64_t height) {
  const at::Device device = geometry.device();
  OrderStage stage;
  stage.count = geometry.size(0);
  stage.order = at::empty({stage.count}, on(device, at::kInt));
  stage.starts = at::empty({stage.count}, on(device, at::kLong));
  stage.rects = at::empty({stage.count, 4}, on(device, at::kInt));
  stage.totals = at::empty({2}, on(device, at::kLong));
  stage.space = workspace(api.bin_order_workspace_size(stage.count), device);
  check(api.bin_order_count(ptr<const float>(geometry), ptr<const int32_t>(radii),
                            ptr<const int64_t>(image_ids), stage.count, int32_t(width),
                            int32_t(height), ptr<int32_t>(stage.rects),
                            ptr<int64_t>(stage.totals), ptr<int64_t>(stage.totals) + 1,
                            stage.space.data_ptr(), size_t(stage.space.numel()),
                            stream_of(device)));
  return stage;
}

// The block path's count stage: stacked rectangles, block counts, and
// totals = (M, V, block entries).
OrderStage count_stage_blocks(const at::Tensor& geometry, const at::Tensor& radii,
                              const at::Tensor& image_ids, int64_t width, int64_t height,
                              double near_plane, double far_plane) {
  const at::Device device = geometry.device();
  OrderStage stage;
  stage.count = geometry.size(0);
  stage.blocks = true;
  stage.near_plane = float(near_plane);
  stage.far_plane = float(far_plane);
  stage.order = at::empty({stage.count}, on(device, at::kInt));
  stage.starts = at::empty({stage.count}, on(device, at::kLong));
  stage.rects = at::empty({stage.count, 4}, on(device, at::kInt));
  stage.totals = at::empty({3}, on(device, at::kLong));
  stage.space = workspace(api.bin_order_workspace_size(stage.count), device);
  check(api.bin_blocks_count(ptr<const float>(geometry), ptr<const int32_t>(radii),
                             ptr<const int64_t>(image_ids), stage.count, int32_t(width),
                             int32_t(height), stage.near_plane, stage.far_plane,
                             ptr<int32_t>(stage.rects), ptr<int64_t>(stage.totals),
                             stage.space.data_ptr(), size_t(stage.space.numel()),
                             stream_of(device)));
  return stage;
}

void sort_stage(OrderStage& stage) {
  void* stream = stream_of(stage.order.device());
  if (stage.blocks)
    check(api.bin_blocks_sort(stage.count, stage.near_plane, stage.far_plane,
                              ptr<int32_t>(stage.order), ptr<int64_t>(stage.starts),
                              stage.space.data_ptr(), size_t(stage.space.numel()), stream));
  else
    check(api.bin_order_sort(stage.count, ptr<int32_t>(stage.order), ptr<int64_t>(stage.starts),
                             stage.space.data_ptr(), size_t(stage.space.numel()), stream));
}

py::tuple bin_order(const at::Tensor& geometry, const at::Tensor& radii,
                    const at::Tensor& image_ids, int64_t width, int64_t height) {
  require_bound();
  c10::DeviceGuard guard(geometry.device());
  OrderStage stage = count_stage(geometry, radii, image_ids, width, height);
  sort_stage(stage);
  return py::make_tuple(stage.order, stage.starts, stage.rects, stage.totals);
}

// Stage 1 of the block path: order, block starts, stacked rectangles and
// totals (M, V, block entries) on the device.
py::tuple bin_blocks_order(const at::Tensor& geometry, const at::Tensor& radii,
                           const at::Tensor& image_ids, int64_t width, int64_t height,
                           double near_plane, double far_plane) {
  require_bound();
  c10::DeviceGuard guard(geometry.device());
  OrderStage stage = count_stage_blocks(geometry, radii, image_ids, width, height, near_plane,
                                        far_plane);
  sort_stage(stage);
  return py::make_tuple(stage.order, stage.starts, stage.rects, stage.totals);
}

// Stage-2 path of the synchronised binning (bin_depth_first without a
// capacity): 0 = the block path wherever the block ids fit
// (gs_bin_blocks_fit), 1 = the tile sort. Process-wide.
std::atomic<int> binning_path{0};

void set_binning_path(const std::string& name) {
  if (name == "blocks") binning_path = 0;
  else if (name == "tiles") binning_path = 1;
  else fail("binning path must be 'blocks' or 'tiles'");
}

std::string get_binning_path() { return binning_path.load() == 0 ? "blocks" : "tiles"; }

std::pair<at::Tensor, at::Tensor> bin_tiles_impl(const at::Tensor& order, const at::Tensor& starts,
                                                 const at::Tensor& rects, int64_t images,
                                                 int64_t width, int64_t height,
                                                 int64_t intersections, int64_t visible,
                                                 const std::optional<at::Tensor>& status) {
  const at::Device device = order.device();
  const int64_t count = order.size(0);
  const int64_t tiles = images * tiles_across(width) * tiles_across(height);
  c10::DeviceGuard guard(device);
  const at::Tensor point_list = at::empty({intersections}, on(device, at::kInt));
  const at::Tensor ranges = at::empty({tiles, 2}, on(device, at::kInt));
  const at::Tensor space = workspace(api.bin_tiles_workspace_size(intersections), device);
  check(api.bin_tiles(ptr<const int32_t>(order), ptr<const int64_t>(starts),
                      ptr<const int32_t>(rects), count, intersections, visible, images,
                      int32_t(width), int32_t(height), ptr<int32_t>(point_list),
                      ptr<int32_t>(ranges), ptr<uint32_t>(status), space.data_ptr(),
                      size_t(space.numel()), stream_of(device)));
  return {point_list, ranges};
}

std::pair<at::Tensor, at::Tensor> bin_blocks_tiles_impl(
    const at::Tensor& order, const at::Tensor& starts, const at::Tensor& rects, int64_t images,
    int64_t width, int64_t height, int64_t intersections, int64_t entries, int64_t visible,
    const std::optional<at::Tensor>& status) {
  const at::Device device = order.device();
  const int64_t count = order.size(0);
  const int64_t tiles = images * tiles_across(width) * tiles_across(height);
  c10::DeviceGuard guard(device);
  const at::Tensor point_list = at::empty({intersections}, on(device, at::kInt));
  const at::Tensor ranges = at::empty({tiles, 2}, on(device, at::kInt));
  const at::Tensor space = workspace(
      api.bin_blocks_tiles_workspace_size(entries, images, int32_t(width), int32_t(height)),
      device);
  check(api.bin_blocks_tiles(ptr<const int32_t>(order), ptr<const int64_t>(starts),
                             ptr<const int32_t>(rects), count, intersections, entries, visible,
                             images, int32_t(width), int32_t(height), ptr<int32_t>(point_list),
                             ptr<int32_t>(ranges), ptr<uint32_t>(status), space.data_ptr(),
                             size_t(space.numel()), stream_of(device)));
  return {point_list, ranges};
}

py::tuple bin_tiles(const at::Tensor& order, const at::Tensor& starts, const at::Tensor& rects,
                    int64_t images, int64_t width, int64_t height, int64_t intersections,
                    int64_t visible, const std::optional<at::Tensor>& status) {
  require_bound();
  auto [point_list, ranges] =
      bin_tiles_impl(order, starts, rects, images, width, height, intersections, visible, status);
  return py::make_tuple(point_list, ranges);
}

py::tuple bin_blocks_tiles(const at::Tensor& order, const at::Tensor& starts,
                           const at::Tensor& rects, int64_t images, int64_t width, int64_t height,
                           int64_t intersections, int64_t entries, int64_t visible,
                           const std::optional<at::Tensor>& status) {
  require_bound();
  auto [point_list, ranges] = bin_blocks_tiles_impl(order, starts, rects, images, width, height,
                                                    intersections, entries, visible, status);
  return py::make_tuple(point_list, ranges);
}

py::tuple bin_tiles_bounded(const at::Tensor& order, const at::Tensor& starts,
                            const at::Tensor& rects, int64_t images, int64_t width,
                            int64_t height, int64_t capacity, const at::Tensor& intersections) {
  require_bound();
  const at::Device device = order.device();
  const int64_t count = order.size(0);
  const int64_t tiles = images * tiles_across(width) * tiles_across(height);
  c10::DeviceGuard guard(device);
  const at::Tensor point_list = at::empty({capacity}, on(device, at::kInt));
  const at::Tensor ranges = at::empty({tiles, 2}, on(device, at::kInt));
  const at::Tensor overflow = at::empty({1}, on(device, at::kInt));
  const at::Tensor space = workspace(api.bin_tiles_workspace_size(capacity), device);
  check(api.bin_tiles_bounded(ptr<const int32_t>(order), ptr<const int64_t>(starts),
                              ptr<const int32_t>(rects), count, capacity,
                              ptr<const int64_t>(intersections), images, int32_t(width),
                              int32_t(height), ptr<int32_t>(point_list), ptr<int32_t>(ranges),
                              ptr<uint32_t>(overflow), space.data_ptr(), size_t(space.numel()),
                              stream_of(device)));
  return py::make_tuple(point_list, ranges, overflow);
}

py::tuple bin_blocks_tiles_bounded(const at::Tensor& order, const at::Tensor& starts,
                                   const at::Tensor& rects, int64_t images, int64_t width,
                                   int64_t height, int64_t capacity, const at::Tensor& totals) {
  require_bound();
  require(totals.numel() >= 3 && totals.scalar_type() == at::kLong && totals.is_contiguous(),
          "totals must be the contiguous int64 (M, V, E) of bin_blocks_order");
  const at::Device device = order.device();
  const int64_t count = order.size(0);
  const int64_t tiles = images * tiles_across(width) * tiles_across(height);
  c10::DeviceGuard guard(device);
  const at::Tensor point_list = at::empty({capacity}, on(device, at::kInt));
  const at::Tensor ranges = at::empty({tiles, 2}, on(device, at::kInt));
  const at::Tensor overflow = at::empty({1}, on(device, at::kInt));
  const at::Tensor space = workspace(
      api.bin_blocks_tiles_workspace_size(capacity, images, int32_t(width), int32_t(height)),
      device);
  check(api.bin_blocks_tiles_bounded(
      ptr<const int32_t>(order), ptr<const int64_t>(starts), ptr<const int32_t>(rects), count,
      capacity, ptr<const int64_t>(totals), images, int32_t(width), int32_t(height),
      ptr<int32_t>(point_list), ptr<int32_t>(ranges), ptr<uint32_t>(overflow), space.data_ptr(),
      size_t(space.numel()), stream_of(device)));
  return py::make_tuple(point_list, ranges, overflow);
}

// Both binning stages with the one host synchronisation for M between them
// (rasterize.cu:466-469). Stage 1's first kernel sums M and V; they are
// copied to pinned host memory right behind it, and the host waits on an
// event recorded after that copy, not on the stream: the depth sort (queued
// before the wait) and GPU work that overlap() queues run during the wait
// (which releases the GIL) and while the host then queues stage 2, so the
// read-back leaves no gap on the GPU. With a capacity there is no
// synchronisation: flags(overflow, total) receives the status word and the
// live count, both on the device. violations = (device int32 word, function
// raising for a nonzero word) is read back with M and reported before M is
// checked or used. Stage 2 takes the block path (gs_bin_blocks_*, which
// also reads the block entry count back with M, or reads it on the device
// with a capacity) whenever the block ids fit, and the tile sort otherwise;
// both give the same point list and ranges.
std::pair<at::Tensor, at::Tensor> bin_depth_first_impl(
    const at::Tensor& geometry, const at::Tensor& radii, const at::Tensor& image_ids,
    int64_t images, int64_t width, int64_t height, const py::object& overlap,
    const std::optional<int64_t>& capacity, const py::object& flags,
    const py::object& violations, double near_plane, double far_plane) {
  const bool blocks = binning_path.load() == 0 &&
                      api.bin_blocks_fit(images, int32_t(width), int32_t(height)) == 1;
  OrderStage stage = blocks ? count_stage_blocks(geometry, radii, image_ids, width, height,
                                                near_plane, far_plane)
                            : count_stage(geometry, radii, image_ids, width, height);
  const at::Tensor total = stage.totals.slice(0, 0, 1);
  if (capacity) {
    sort_stage(stage);
    if (!overlap.is_none()) overlap();
    const py::tuple bounded =
        blocks ? bin_blocks_tiles_bounded(stage.order, stage.starts, stage.rects, images, width,
                                          height, *capacity, stage.totals)
               : bin_tiles_bounded(stage.order, stage.starts, stage.rects, images, width,
                                   height, *capacity, total);
    if (!flags.is_none()) flags(bounded[2], total);
    return {bounded[0].cast<at::Tensor>(), bounded[1].cast<at::Tensor>()};
  }
  const at::Device device = geometry.device();
  hipStream_t stream = static_cast<hipStream_t>(stream_of(device));
  Readback& state = readback();
  const hipEvent_t ready = readback_event(state, device);
  check_hip(hipMemcpyAsync(state.host, stage.totals.data_ptr(),
                           size_t(stage.totals.numel()) * sizeof(int64_t),
                           hipMemcpyDeviceToHost, stream),
            "hipMemcpyAsync");
  at::Tensor word;
  py::object report;
  if (!violations.is_none()) {
    const py::tuple pending = violations.cast<py::tuple>();
    word = pending[0].cast<at::Tensor>();
    report = pending[1];
    check_hip(hipMemcpyAsync(state.host + 3, word.data_ptr(), sizeof(int32_t),
                             hipMemcpyDeviceToHost, stream),
              "hipMemcpyAsync");
  }
  check_hip(hipEventRecord(ready, stream), "hipEventRecord");
  auto wait = [ready] {
    py::gil_scoped_release released;
    return hipEventSynchronize(ready);
  };
  try {
    sort_stage(stage);
    if (!overlap.is_none()) overlap();
  } catch (...) {
    // The copy into this thread's pinned buffer must land before the
    // buffer can be reused by a later call, possibly on another stream.
    wait();
    throw;
  }
  check_hip(wait(), "hipEventSynchronize");
  const int64_t intersections = state.host[0], visible = state.host[1];
  const int64_t entries = blocks ? state.host[2] : 0;
  if (word.defined()) {
    const int32_t value = *reinterpret_cast<const int32_t*>(state.host + 3);
    report(value);
  }
  require(intersections <= kIntMax, "tile intersection count exceeds int32");
  if (blocks)
    return bin_blocks_tiles_impl(stage.order, stage.starts, stage.rects, images, width, height,
                                 intersections, entries, visible, std::nullopt);
  return bin_tiles_impl(stage.order, stage.starts, stage.rects, images, width, height,
                        intersections, visible, std::nullopt);
}

py::tuple bin_depth_first(const at::Tensor& geometry, const at::Tensor& radii,
                          const at::Tensor& image_ids, int64_t images, int64_t width,
                          int64_t height, const py::object& overlap,
                          const std::optional<int64_t>& capacity, const py::object& flags,
                          const py::object& violations, double near_plane, double far_plane) {
  require_bound();
  c10::DeviceGuard guard(geometry.device());
  auto [point_list, ranges] =
      bin_depth_first_impl(geometry, radii, image_ids, images, width, height, overlap, capacity,
                           flags, violations, near_plane, far_plane);
  return py::make_tuple(point_list, ranges);
}

// --------------------------------------------------------------------------
// Compositor operators (the reference's _C.rasterize_forward / backward).

// (pixel stride, channel stride) in elements when every pixel of the
// [I,H,W,k] tensor sits at p * pixel_stride from its first element,
// p = (i*H + y)*W + x; nullopt otherwise.
std::optional<std::pair<int64_t, int64_t>> flat_pixel_stride(const at::Tensor& t) {
  const auto sizes = t.sizes();
  const auto strides = t.strides();
  const int64_t dims = t.dim();
  const int64_t k = sizes[dims - 1];
  std::optional<int64_t> stride;
  int64_t inner = 1;
  for (int64_t d = dims - 2; d >= 0; --d) {
    const int64_t size = sizes[d], step = strides[d];
    if (size > 1) {
      if (!stride) stride = step % inner == 0 ? step / inner : -1;
      if (*stride < 0 || step != *stride * inner) return std::nullopt;
    }
    inner *= size;
  }
  return std::make_pair(stride.value_or(0), k > 1 ? strides[dims - 1] : int64_t(0));
}

struct MapArgs {
  std::array<float*, 5> data{};
  std::array<int64_t, 10> strides{};
};

MapArgs map_group_args(const std::array<at::Tensor, 5>& groups, const char* message) {
  MapArgs args;
  for (int g = 0; g < 5; ++g) {
    if (!groups[g].defined()) continue;
    const auto layout = flat_pixel_stride(groups[g]);
    require(layout.has_value(), message);
    args.data[g] = ptr<float>(groups[g]);
    args.strides[2 * g] = layout->first;
    args.strides[2 * g + 1] = layout->second;
  }
  return args;
}

std::array<at::Tensor, 5> split_map_groups(const at::Tensor& maps) {
  std::array<at::Tensor, 5> groups;
  int64_t first = 0;
  for (int g = 0; g < 5; ++g) {
    groups[g] = maps.slice(-1, first, first + kMapGroups[g]);
    first += kMapGroups[g];
  }
  return groups;
}

int64_t split_index_length(int64_t tiles, int64_t slots) {
  return (tiles + slots + 1) / 2 * 2 + 2 * (tiles + slots);
}

py::list rasterize_forward(const at::Tensor& geometry, const at::Tensor& appearance,
                           const at::Tensor& opacities, const at::Tensor& primitive_ids,
                           const at::Tensor& image_ids, const at::Tensor& radii,
                           const at::Tensor& backgrounds, int64_t width, int64_t height,
                           bool neural, double near_plane, double far_plane,
                           const py::object& outputs, const py::object& overlap,
                           const std::optional<int64_t>& capacity, const py::object& flags,
                           bool replay, const py::object& violations, int64_t split,
                           int64_t split_max_tiles, int64_t split_length,
                           int64_t split_max_slots) {
  require_bound();
  check_buffers(geometry, appearance, opacities, primitive_ids, backgrounds, neural);
  require(0 < width && width < kIntMax - kTile && 0 < height && height < kIntMax - kTile,
          "invalid image dimensions");
  require(near_plane > 0 && far_plane > near_plane, "invalid clipping planes");
  require(image_ids.device() == geometry.device() && image_ids.is_contiguous() &&
              image_ids.scalar_type() == at::kLong && image_ids.dim() == 1 &&
              image_ids.size(0) == geometry.size(0),
          "invalid image IDs");
  require(radii.device() == geometry.device() && radii.is_contiguous() &&
              radii.scalar_type() == at::kInt && radii.dim() == 1 &&
              radii.size(0) == geometry.size(0),
          "invalid radii");
  const at::Device device = geometry.device();
  c10::DeviceGuard guard(device);
  void* stream = stream_of(device);
  const int64_t images = backgrounds.size(0);
  const int64_t tiles = images * tiles_across(width) * tiles_across(height);
  require(tiles <= kIntMax, "image tile count exceeds int32");
  const auto f32 = on(device, at::kFloat);
  const auto i32 = on(device, at::kInt);
  const at::Tensor state = at::empty({images, height, width, 3}, f32);
  const at::Tensor contributors = at::empty({images, height, width}, i32);
  auto [point_list, ranges] =
      bin_depth_first_impl(geometry, radii, image_ids, images, width, height, overlap, capacity,
                           flags, violations, near_plane, far_plane);
  std::array<at::Tensor, 5> groups;
  py::object maps;
  if (outputs.is_none()) {
    const at::Tensor all = at::empty({images, height, width, kMapSize}, f32);
    groups = split_map_groups(all);
    maps = py::cast(all);
  } else {
    const py::sequence given(outputs);
    bool ok = py::len(given) == 5;
    for (int g = 0; ok && g < 5; ++g) {
      groups[g] = given[g].cast<at::Tensor>();
      ok = same_shape(groups[g], {images, height, width, kMapGroups[g]}) &&
           groups[g].scalar_type() == at::kFloat && groups[g].device() == device;
    }
    require(ok, "invalid map outputs");
    maps = py::tuple(given);
  }
  const MapArgs args = map_group_args(groups, "map outputs must have uniformly strided pixels");
  const int64_t m = point_list.numel();
  int64_t length = split >= 0 ? split : ((tiles >= split_max_tiles || m <= 0) ? 0 : split_length);
  // A tile of L > length records takes ceil(L / length) <= floor(L / length) + 1
  // slots, and at most min(tiles, m / (length + 1)) tiles are that long.
  const int64_t slots =
      length ? std::min(m / length + std::min(tiles, m / (length + 1)) + 1, split_max_slots) : 0;
  at::Tensor segment_state, segment_index;
  if (slots) {
    segment_state = at::empty({slots, kCheckpointFloats, kTile * kTile}, f32);
    segment_index = at::empty({split_index_length(tiles, slots)}, i32);
  } else {
    length = 0;
  }
  at::Tensor entries, counts;
  py::object lists = py::none();
  if (replay && m < kReplayMaxEntries) {
    entries = at::empty({std::max<int64_t>(m, 1), 2}, i32);
    counts = at::empty({tiles}, i32);
    py::object segments = py::none();
    if (slots) segments = py::make_tuple(length, segment_state, segment_index);
    lists = py::make_tuple(entries, counts, segments);
  }
  const at::Tensor space = workspace(api.render_workspace_size(images, int32_t(width),
                                                               int32_t(height)),
                                     device);
  check(api.render_forward(
      neural ? 1 : 0, ptr<const float>(geometry), ptr<const float>(appearance),
      ptr<const float>(opacities), ptr<const int64_t>(primitive_ids),
      ptr<const float>(backgrounds), ptr<const int32_t>(point_list), ptr<const int32_t>(ranges),
      images, int32_t(width), int32_t(height), float(near_plane), float(far_plane),
      args.data.data(), args.strides.data(), ptr<float>(state), ptr<int32_t>(contributors),
      ptr<int32_t>(entries), m, ptr<int32_t>(counts), int32_t(length), ptr<float>(segment_state),
      ptr<int32_t>(segment_index), slots, space.data_ptr(), size_t(space.numel()), stream));
  py::list result;
  result.append(maps);
  result.append(point_list);
  result.append(ranges);
  result.append(state);
  result.append(contributors);
  if (replay) result.append(lists);
  return result;
}

// Zeroed accumulators shaped like (geometry, appearance, opacities,
// backgrounds). `appearance` is one tensor, or a sequence of tensors (the
// neural renderer's SIREN parameter groups), whose accumulator is then a
// tuple of the same shapes.
py::tuple zero_accumulators(const at::Tensor& geometry, const py::object& appearance,
                            const at::Tensor& opacities, const at::Tensor& backgrounds,
                            bool shared) {
  std::vector<at::Tensor> appearance_like;
  const bool grouped = !THPVariable_Check(appearance.ptr());
  if (grouped) {
    for (const py::handle item : py::sequence(appearance))
      appearance_like.push_back(item.cast<at::Tensor>());
  } else {
    appearance_like.push_back(appearance.cast<at::Tensor>());
  }
  std::vector<const at::Tensor*> like = {&geometry};
  for (const at::Tensor& t : appearance_like) like.push_back(&t);
  like.push_back(&opacities);
  like.push_back(&backgrounds);
  c10::DeviceGuard guard(geometry.device());
  std::vector<at::Tensor> made;
  if (!shared) {
    for (const at::Tensor* t : like) made.push_back(at::zeros_like(*t));
  } else {
    int64_t total = 0;
    for (const at::Tensor* t : like) total += t->numel();
    const at::Tensor flat = at::zeros({total}, on(geometry.device(), at::kFloat));
    int64_t first = 0;
    for (const at::Tensor* t : like) {
      const int64_t size = t->numel();
      made.push_back(flat.slice(0, first, first + size).view(t->sizes()));
      first += size;
    }
  }
  const size_t n = appearance_like.size();
  py::object appearance_grads = py::cast(made[1]);
  if (grouped) {
    py::tuple columns(n);
    for (size_t g = 0; g < n; ++g) columns[g] = made[1 + g];
    appearance_grads = columns;
  }
  return py::make_tuple(made[0], appearance_grads, made[1 + n], made[2 + n]);
}

py::list rasterize_backward(const at::Tensor& geometry, const at::Tensor& appearance,
                            const at::Tensor& opacities, const at::Tensor& primitive_ids,
                            const at::Tensor& backgrounds, const at::Tensor& point_list,
                            const at::Tensor& ranges, const at::Tensor& state,
                            const at::Tensor& contributors, const py::object& grad_maps,
                            int64_t width, int64_t height, bool neural, double near_plane,
                            double far_plane, const py::object& accumulators,
                            const py::object& replay) {
  require_bound();
  check_buffers(geometry, appearance, opacities, primitive_ids, backgrounds, neural);
  const at::Device device = geometry.device();
  const int64_t images = backgrounds.size(0);
  std::array<at::Tensor, 5> groups;
  if (THPVariable_Check(grad_maps.ptr())) {
    const at::Tensor all = grad_maps.cast<at::Tensor>();
    check_float(all, geometry);
    require(same_shape(all, {images, height, width, kMapSize}), "invalid map gradient");
    groups = split_map_groups(all);
  } else {
    const py::sequence given(grad_maps);
    bool ok = py::len(given) == 5;
    for (int g = 0; ok && g < 5; ++g) {
      if (given[g].is_none()) continue;
      groups[g] = given[g].cast<at::Tensor>();
      ok = same_shape(groups[g], {images, height, width, kMapGroups[g]}) &&
           groups[g].scalar_type() == at::kFloat && groups[g].device() == device;
    }
    require(ok, "invalid map gradient");
  }
  require(same_shape(state, {images, height, width, 3}) &&
              same_shape(contributors, {images, height, width}),
          "invalid saved compositor state");
  int64_t length = 0, slots = 0;
  at::Tensor segment_state, segment_index, lists, counts;
  if (!replay.is_none()) {
    const py::sequence given(replay);
    lists = given[0].cast<at::Tensor>();
    counts = given[1].cast<at::Tensor>();
    const int64_t tiles = images * tiles_across(width) * tiles_across(height);
    if (py::len(given) > 2 && !given[2].is_none()) {
      const py::sequence segments(given[2]);
      length = segments[0].cast<int64_t>();
      segment_state = segments[1].cast<at::Tensor>();
      segment_index = segments[2].cast<at::Tensor>();
      slots = segment_state.size(0);
      require(segment_state.scalar_type() == at::kFloat &&
                  segment_index.scalar_type() == at::kInt && segment_state.device() == device &&
                  segment_index.device() == device && segment_state.is_contiguous() &&
                  segment_index.is_contiguous() && segment_state.dim() == 3 &&
                  segment_state.size(1) == kCheckpointFloats &&
                  segment_state.size(2) == kTile * kTile &&
                  same_shape(segment_index, {split_index_length(tiles, slots)}),
              "invalid split-tile checkpoints");
    }
    require(lists.scalar_type() == at::kInt && counts.scalar_type() == at::kInt &&
                lists.device() == device && counts.device() == device &&
                lists.is_contiguous() && counts.is_contiguous() && lists.dim() == 2 &&
                lists.size(1) == 2 && lists.size(0) >= point_list.numel() &&
                same_shape(counts, {tiles}),
            "invalid replay lists");
  }
  c10::DeviceGuard guard(device);
  // grads[1] is the appearance rows' gradient, unless the accumulators give
  // the neural appearance's gradient as the SIREN's four parameter groups
  // (column_grads: input weights [P,30], input biases [P,6], output weights
  // [P,18], output biases [P,3]), which the kernel then writes directly.
  std::array<at::Tensor, 4> grads;
  std::array<at::Tensor, 4> column_grads;
  bool columns = false;
  if (accumulators.is_none()) {
    grads = {at::zeros_like(geometry), at::zeros_like(appearance), at::zeros_like(opacities),
             at::zeros_like(backgrounds)};
  } else {
    const py::sequence given(accumulators);
    require(py::len(given) == 4, "invalid gradient accumulators");
    for (int i : {0, 2, 3}) grads[i] = given[i].cast<at::Tensor>();
    columns = !THPVariable_Check(py::object(given[1]).ptr());
    if (columns) {
      const py::sequence groups_given(given[1]);
      require(neural && py::len(groups_given) == 4, "invalid gradient accumulators");
      for (int g = 0; g < 4; ++g) column_grads[g] = groups_given[g].cast<at::Tensor>();
    } else {
      grads[1] = given[1].cast<at::Tensor>();
    }
  }
  constexpr std::array<int64_t, 4> kSirenWidths = {30, 6, 18, 3};
  const int64_t primitives = appearance.size(0);
  bool ok = grads[0].sizes() == geometry.sizes() && grads[2].sizes() == opacities.sizes() &&
            grads[3].sizes() == backgrounds.sizes();
  std::vector<const at::Tensor*> all = {&grads[0], &grads[2], &grads[3]};
  std::array<float*, 4> column_pointers{};
  if (columns) {
    for (int g = 0; g < 4; ++g) {
      ok = ok && same_shape(column_grads[g], {primitives, kSirenWidths[g]});
      all.push_back(&column_grads[g]);
    }
  } else {
    ok = ok && grads[1].sizes() == appearance.sizes();
    all.push_back(&grads[1]);
  }
  for (const at::Tensor* t : all)
    ok = ok && t->is_contiguous() && t->scalar_type() == at::kFloat && t->device() == device;
  require(ok, "invalid gradient accumulators");
  if (columns)
    for (int g = 0; g < 4; ++g) column_pointers[g] = ptr<float>(column_grads[g]);
  for (at::Tensor& g : groups)
    if (g.defined() && !flat_pixel_stride(g)) g = g.contiguous();
  const MapArgs args = map_group_args(groups, "map gradients must have uniformly strided pixels");
  const at::Tensor space = workspace(
      api.render_backward_workspace_size(images, int32_t(width), int32_t(height), slots), device);
  check(api.render_backward(
      neural ? 1 : 0, ptr<const float>(geometry), ptr<const float>(appearance),
      ptr<const float>(opacities), ptr<const int64_t>(primitive_ids),
      ptr<const float>(backgrounds), ptr<const int32_t>(point_list), ptr<const int32_t>(ranges),
      ptr<const float>(state), ptr<const int32_t>(contributors), ptr<const int32_t>(lists),
      ptr<const int32_t>(counts), int32_t(length), ptr<const float>(segment_state),
      ptr<const int32_t>(segment_index), slots,
      const_cast<const float* const*>(args.data.data()), args.strides.data(), images,
      int32_t(width), int32_t(height), float(near_plane), float(far_plane), ptr<float>(grads[0]),
      columns ? nullptr : ptr<float>(grads[1]), columns ? column_pointers.data() : nullptr,
      ptr<float>(grads[2]), ptr<float>(grads[3]), space.data_ptr(), size_t(space.numel()),
      stream_of(device)));
  py::list result;
  result.append(grads[0]);
  if (columns)
    result.append(py::make_tuple(column_grads[0], column_grads[1], column_grads[2],
                                 column_grads[3]));
  else
    result.append(grads[1]);
  result.append(grads[2]);
  result.append(grads[3]);
  return result;
}

}  // namespace

PYBIND11_MODULE(_host, m) {
  m.doc() = "C++ host functions of the renderer over the gfx950 library's C ABI";
  m.def("bind", &bind, py::arg("table"));
  m.def("entry_points", &entry_points);
  m.def("check_tensors", &check_tensors, py::arg("tensors"), py::arg("device"));
  m.def("check_values_word", &check_values_word);
  m.def("pack_visible", &pack_visible, py::arg("radii"), py::arg("with_rows"),
        py::arg("sync"));
  m.def("records_forward", &records_forward);
  m.def("records_backward", &records_backward);
  m.def("bin_order", &bin_order);
  m.def("bin_tiles", &bin_tiles);
  m.def("bin_tiles_bounded", &bin_tiles_bounded);
  m.def("bin_blocks_tiles_bounded", &bin_blocks_tiles_bounded);
  m.def("bin_blocks_order", &bin_blocks_order);
  m.def("bin_blocks_tiles", &bin_blocks_tiles);
  m.def("set_binning_path", &set_binning_path);
  m.def("binning_path", &get_binning_path);
  m.def("bin_depth_first", &bin_depth_first);
  m.def("rasterize_forward", &rasterize_forward);
  m.def("zero_accumulators", &zero_accumulators);
  m.def("rasterize_backward", &rasterize_backward);
}
