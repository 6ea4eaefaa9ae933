"""C++ header emission for generated models.

The reference's generator writes one C++ header per model: a class with the
model's schema, its weights-file loader, its parameter API, a per-sample
`infer_one` and the batch `infer_batch` / `infer_batch_half2` whose bodies
are the model's own kernels (kokkos_nn/emitter.py:1428-1953).  This module
writes the same class surface for a graph (ponni_amd/graph.py) over this
repository's pieces:

- the linearized layer chain as C-ABI descriptors, and per layer a gather
  table from the weights-file storage to the layer's parameter vector;
- the FUSED (or generated NARROW) kernels of the model's fp32/fp64 plan and of
  its fp16 plan, as HIP source compiled AHEAD OF TIME with the application
  (the hipRTC path compiles the same text at run time); `infer_batch` and
  `infer_batch_half2` launch them on the plan's packed parameters;
- `infer_one` over the plan's device description (ponni/device.h).

Build the application with
  hipcc -std=c++17 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops
        -I<repo>/include -I<repo>/ponni_amd/include -I<repo>/ponni_amd/csrc app.cpp
        -L<repo>/ponni_amd -lponni_hip

The header sets `#pragma clang fp contract(on)` before its first include,
so its kernels (and everything after it in the translation unit) fuse
multiply-adds only within one expression: each layer's state is rounded
before the next layer reads it, as in the library's fp32 / fp64 kernels
(-ffp-contract=on), whatever contraction the application compiles with.  It
must therefore come before any other include of ponni.h.
"""
from __future__ import annotations

import re

import numpy as np

from . import _abi as A
from .graph import GeneratedModel, Graph

_BIG = float(2 ** 40)  # storage index i is encoded as _BIG + i while tracing gathers


def _gather_tables(gm: GeneratedModel):
    """Per layer, the storage index (>= 0) or literal (-(k + 1) into literals)
    of every parameter element, found by running each layer's parameter
    builder on constants whose values are their own storage indices (the
    builders only transpose, concatenate, broadcast and pad)."""
    consts = {}
    for cname, tname in gm._name_of_constant.items():
        off = gm._offset[tname]
        shape = gm.graph.constants[cname].values.shape
        n = int(np.prod(shape, dtype=np.int64)) if shape else 1
        v = np.arange(n, dtype=np.float64) + off + _BIG
        consts[cname] = v.reshape(shape) if shape else v
    literals: list[float] = []
    lit_index: dict[float, int] = {}
    tables = []
    for vals in gm.lowered.layer_params(consts):
        t = []
        for x in np.asarray(vals, dtype=np.float64).reshape(-1):
            if x >= _BIG / 2:
                if x != np.floor(x) or x - _BIG >= gm.storage_parameter_elements:
                    raise ValueError("a parameter builder computed with a stored value; no gather table exists")
                t.append(int(x - _BIG))
            elif abs(x) >= _BIG / 2:
                raise ValueError("a parameter builder computed with a stored value; no gather table exists")
            else:
                k = lit_index.setdefault(float(x), len(literals))
                if k == len(literals):
                    literals.append(float(x))
                t.append(-(k + 1))
        tables.append(t)
    return tables, literals


def _kernel_text(src: str) -> str:
    """A generated kernel's source without its includes and C linkage, so it
    can live in a namespace of the application's translation unit."""
    out = []
    for line in src.splitlines():
        if line.startswith("#include"):
            continue
        out.append(line.replace('extern "C" __global__', "__global__"))
    return "\n".join(out)


def _kernel_name(src: str) -> str:
    m = re.search(r"void (ponni_(?:fused|narrow)_\w+)\(", src)
    if not m:
        raise ValueError("no generated kernel in the source")
    return m.group(1)


def _cstr(s: str) -> str:
    return '"' + s.replace("\\", "\\\\").replace('"', '\\"') + '"'


def emit_cpp_header(graph: Graph, path: str, namespace: str = "ponni::generated",
                    class_name: str = "GeneratedModel") -> str:
    """Write the model's C++ header to `path` and return its text."""
    gm = GeneratedModel(graph)
    scalar = "double" if gm.scalar == "f64" else "float"
    tables, literals = _gather_tables(gm)
    layers = gm.lowered.layers

    kernels = {}
    for dt in (gm.scalar, "f16"):
        plan = gm.plan(dt)
        if plan.path in ("fused", "narrow"):
            try:
                threads, cols, persistent = plan.kernel_config()
            except A.PonniError:
                continue  # NARROW with run-time compilation off: the library launches it
            src = plan.kernel_source()
            kernels[dt] = dict(src=_kernel_text(src), name=_kernel_name(src), threads=threads, cols=cols,
                               persistent=persistent, path=plan.path)
    program = gm.plan(gm.scalar).program_source()
    includes = set()
    for k in kernels.values():
        includes.add("narrow_jit.h" if k["path"] == "narrow" else None)
    need_fused = any(k["path"] == "fused" for k in kernels.values())

    o = []
    w = o.append
    w(f"// Generated by ponni_amd.emitter.emit_cpp_header for model {gm.model_fingerprint()}.")
    w("// The class surface of the reference generator's header (kokkos_nn/emitter.py:1589-1953)")
    w("// over libponni_hip; the model's kernels below are compiled with the application.")
    w("// hipcc -std=c++17 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops")
    w("//       -I<repo>/include -I<repo>/ponni_amd/include -I<repo>/ponni_amd/csrc ... -lponni_hip")
    w("#pragma once")
    w("")
    w("// Kernels below and the helpers they inline fuse multiply-adds only within one expression,")
    w("// so a layer's state is rounded before the next layer reads it (the library compiles its")
    w("// fp32 / fp64 kernels the same way).  The rule applies from here to the end of the")
    w("// translation unit; the helpers are compiled at their first include, hence the check.")
    w("#if defined(PONNI_POINTWISE_H) && !defined(PONNI_GENERATED_CONTRACT_ON)")
    w('#error "include the generated model header before ponni.h and the library kernel headers"')
    w("#endif")
    w("#pragma clang fp contract(on)")
    w("#define PONNI_GENERATED_CONTRACT_ON 1")
    w("")
    w('#include "ponni.h"')
    if need_fused:
        w('#include "fused_f16.h"')
    if "narrow_jit.h" in includes:
        w('#include "narrow_jit.h"')
    w("")
    w("#include <algorithm>")
    w("#include <cmath>")
    w("#include <cstdint>")
    w("#include <memory>")
    w("#include <string>")
    w("#include <vector>")
    w("")
    ns_open = "".join(f"namespace {p} {{ " for p in namespace.split("::"))
    ns_close = "".join("} " for _ in namespace.split("::"))
    w(ns_open)
    w("")
    w("// Occupancy targets of the kernels are upper bounds, settled when the library compiled them.")
    w("#pragma clang diagnostic push")
    w('#pragma clang diagnostic ignored "-Wpass-failed"')
    w(f"namespace {class_name}_kernels {{")
    for dt, k in kernels.items():
        w(f"namespace k_{dt} {{")
        w(k["src"])
        w(f"}}  // namespace k_{dt}")
    w(f"}}  // namespace {class_name}_kernels")
    w("#pragma clang diagnostic pop")
    w("")
    w(f"class {class_name} {{")
    w(" public:")
    w(f"  using Scalar = {scalar};")
    w(f"  static constexpr int num_inputs = {gm.num_inputs};")
    w(f"  static constexpr int num_outputs = {gm.num_outputs};")
    w(f"  static constexpr std::int64_t storage_parameter_elements = {gm.storage_parameter_elements};")
    w(f"  static constexpr std::int64_t learned_parameter_elements = {gm.learned_parameter_elements};")
    w(f"  static constexpr int stored_scalar_bytes = {8 if gm.scalar == 'f64' else 4};")
    w("  using scalar_type = Scalar;")
    w("  using InputView = ponni::View<Scalar>;")
    w("  using OutputView = ponni::View<Scalar>;")
    w("")
    w("  struct WeightSpec {")
    w("    char const* name;")
    w("    char const* dtype;")
    w("    int rank;")
    w("    std::int64_t shape[8];")
    w("    std::int64_t offset;")
    w("  };")
    w("  // Tensors of weights.ponni in storage order (names sorted), emitter.py:1438-1447.")
    w("  static std::vector<WeightSpec> weight_specs() {")
    w("    return {")
    for s in gm.weight_specs():
        shape = ", ".join(str(d) for d in s.shape) or "0"
        w(f"        {{{_cstr(s.name)}, {_cstr(s.dtype)}, {len(s.shape)}, {{{shape}}}, {s.offset}}},")
    w("    };")
    w("  }")
    w(f"  static std::string model_fingerprint() {{ return {_cstr(gm.model_fingerprint())}; }}")
    w("")
    w("  // Learned-parameter index -> storage index (emitter.py:1454-1465).")
    w("  static std::int64_t parameter_storage_index(std::int64_t index) {")
    w("    static constexpr std::int64_t ranges[][3] = {")
    for lo, so, n in gm._learned_ranges:
        w(f"        {{{lo}, {so}, {n}}},")
    if not gm._learned_ranges:
        w("        {0, 0, 0},")
    w("    };")
    w("    for (auto const& r : ranges)")
    w("      if (index < r[0] + r[2]) return r[1] + index - r[0];")
    w('    ponni::abort("GeneratedModel learned parameter index is out of range");')
    w("  }")
    w("")
    w("  // Copies share the weights, plans and buffers (the reference's generated model")
    w("  // holds Kokkos Views, which copy shallowly): a copy taken before load_weights or")
    w("  // set_parameters sees them, and a copy may be captured by value in a kernel.")
    w(f"  explicit {class_name}(hipStream_t stream = nullptr) : state_(std::make_shared<State>()) {{")
    w("    state_->stream = stream;")
    w("    state_->storage.assign(static_cast<std::size_t>(storage_parameter_elements), 0.0);")
    w("    state_->loaded = storage_parameter_elements == 0;")
    w("    state_->scalar = make_plan(" + ("PONNI_F64" if scalar == "double" else "PONNI_F32") + ");")
    w("    state_->half = make_plan(PONNI_F16);")
    w("    push(state_->scalar.get());")
    w("    push(state_->half.get());")
    w("  }")
    w("")
    w("  static constexpr int get_num_parameters() { return static_cast<int>(learned_parameter_elements); }")
    w("")
    w("  // ---- weights (emitter.py:1724-1766) ----")
    w("  bool load_weights(std::string const& path, std::string* error = nullptr) {")
    w("    std::vector<ponni_tensor_spec> specs = cspecs();")
    w("    std::vector<double> st(static_cast<std::size_t>(storage_parameter_elements));")
    w("    int const rc = ponni_file_read_tensors(path.c_str(), model_fingerprint().c_str(), specs.data(),")
    w("                                           static_cast<int>(specs.size()), st.data(), stored_scalar_bytes);")
    w("    if (rc != PONNI_OK) {")
    w("      if (error) *error = ponni_last_error();")
    w("      return false;")
    w("    }")
    w("    state_->storage = std::move(st);")
    w("    state_->loaded = true;")
    w("    push(state_->scalar.get());")
    w("    push(state_->half.get());")
    w("    return true;")
    w("  }")
    w("  bool save_parameters(std::string const& path, std::string* error = nullptr) const {")
    w("    if (!state_->loaded) {")
    w('      if (error) *error = "generated model parameters are not loaded";')
    w("      return false;")
    w("    }")
    w("    std::vector<ponni_tensor_spec> specs = cspecs();")
    w("    int const rc = ponni_file_write_tensors(path.c_str(), model_fingerprint().c_str(), specs.data(),")
    w("                                            static_cast<int>(specs.size()), state_->storage.data(), stored_scalar_bytes,")
    w('                                            "ponni", "generated");')
    w("    if (rc != PONNI_OK) {")
    w("      if (error) *error = ponni_last_error();")
    w("      return false;")
    w("    }")
    w("    return true;")
    w("  }")
    w("  bool weights_loaded() const { return state_->loaded; }")
    w("")
    w("  // ---- parameters (emitter.py:1768-1895): learned order, host vectors or device views ----")
    w("  template <class T>")
    w("  void get_parameters(std::vector<T>& destination) const {")
    w('    if (!state_->loaded) ponni::abort("GeneratedModel::get_parameters called before load_weights");')
    w("    if (static_cast<std::int64_t>(destination.size()) != learned_parameter_elements)")
    w('      ponni::abort("GeneratedModel::get_parameters destination extent is incorrect");')
    w("    for (std::int64_t i = 0; i < learned_parameter_elements; i++)")
    w("      destination[i] = static_cast<T>(static_cast<Scalar>(state_->storage[parameter_storage_index(i)]));")
    w("  }")
    w("  // Device views: any [1, n] or [n, 1] ponni::View holding the n learned parameters.")
    w("  template <class T>")
    w("  void get_parameters(ponni::View<T> const& destination) const {")
    w("    std::vector<T> v(static_cast<std::size_t>(destination.size()));")
    w("    get_parameters(v);")
    w("    destination.copy_from_host(v);")
    w("  }")
    w("  template <class T>")
    w("  void set_parameters(std::vector<T> const& source) {")
    w('    if (!state_->loaded) ponni::abort("GeneratedModel::set_parameters called before load_weights");')
    w("    if (static_cast<std::int64_t>(source.size()) != learned_parameter_elements)")
    w('      ponni::abort("GeneratedModel::set_parameters source extent is incorrect");')
    w("    for (std::int64_t i = 0; i < learned_parameter_elements; i++)")
    w("      state_->storage[parameter_storage_index(i)] = static_cast<Scalar>(source[i]);")
    w("    push(state_->scalar.get());")
    w("    push(state_->half.get());")
    w("  }")
    w("  template <class T>")
    w("  void set_parameters(ponni::View<T> const& source) {")
    w("    set_parameters(source.copy_to_host());")
    w("  }")
    w("  // The fp16 copy follows every parameter change already; kept for the API.")
    w("  void refresh_half_parameters() {")
    w('    if (!state_->loaded) ponni::abort("GeneratedModel::refresh_half_parameters called before load_weights");')
    w("    push(state_->half.get());")
    w("  }")
    w("  bool parameters_are_finite() const {")
    w("    if (!state_->loaded) return false;")
    w("    for (std::int64_t i = 0; i < learned_parameter_elements; i++)")
    w("      if (!std::isfinite(static_cast<Scalar>(state_->storage[parameter_storage_index(i)]))) return false;")
    w("    return true;")
    w("  }")
    w("  bool parameters_synchronized() const { return state_->loaded; }")
    w("")
    w("  // ---- inference ----")
    w("  // x [num_inputs, B], y [num_outputs, B]: LayoutRight device views of Scalar.")
    w("  template <class InputViewType, class OutputViewType>")
    w("  void infer_batch(InputViewType const& x, OutputViewType const& y) const {")
    w("    ponni::require_layout_right_views<InputViewType, OutputViewType>();")
    w("    std::int64_t const batch = checked_batch(x, y);")
    if gm.scalar in kernels:
        k = kernels[gm.scalar]
        w(f"    launch({class_name}_kernels::k_{gm.scalar}::{k['name']}, {k['threads']}, {k['cols']}, "
          f"{'true' if k['persistent'] else 'false'}, state_->scalar.get(), x.data(), x.stride(0), y.data(), y.stride(0), batch);")
    else:
        w("    ponni::check(ponni_forward(state_->scalar.get(), x.data(), x.stride(0), y.data(), y.stride(0), batch, state_->stream),")
        w('                 "infer_batch");')
    w("  }")
    w("")
    w("  // fp16 operands, fp32 accumulation, on Scalar views (emitter.py:1551-1573).")
    w("  template <class InputViewType, class OutputViewType>")
    w("  void infer_batch_half2(InputViewType const& x, OutputViewType const& y) const {")
    w("    ponni::require_layout_right_views<InputViewType, OutputViewType>();")
    w("    std::int64_t const batch = checked_batch(x, y);")
    w("    half_buffers(batch);")
    w("    unsigned const blocks_in = static_cast<unsigned>((num_inputs * batch + 255) / 256);")
    w("    hipLaunchKernelGGL((convert_rows<Scalar, _Float16>), dim3(blocks_in), dim3(256), 0, state_->stream, x.data(),")
    w("                       static_cast<std::int64_t>(x.stride(0)), state_->hx, batch, num_inputs * batch, batch);")
    if "f16" in kernels:
        k = kernels["f16"]
        w(f"    launch({class_name}_kernels::k_f16::{k['name']}, {k['threads']}, {k['cols']}, "
          f"{'true' if k['persistent'] else 'false'}, state_->half.get(), state_->hx, batch, state_->hy, batch, batch);")
    else:
        w("    ponni::check(ponni_forward(state_->half.get(), state_->hx, batch, state_->hy, batch, batch, state_->stream), \"infer_batch_half2\");")
    w("    unsigned const blocks_out = static_cast<unsigned>((num_outputs * batch + 255) / 256);")
    w("    hipLaunchKernelGGL((convert_rows<_Float16, Scalar>), dim3(blocks_out), dim3(256), 0, state_->stream, state_->hy, batch,")
    w("                       y.data(), static_cast<std::int64_t>(y.stride(0)), num_outputs * batch, batch);")
    w("  }")
    w("")
    w("  // The model's per-sample program (the library's GENERIC lowering of it), fixed at")
    w("  // compile time: infer_one expands every op in place, with thread-private states")
    w("  // sized to the model (the reference's planned local storage).")
    w("  struct program {")
    for line in program.rstrip("\n").split("\n"):
        w("  " + line)
    w("  };")
    w("")
    w("  // One sample inside an application kernel (emitter.py:1897-1901): capture a copy")
    w("  // of the model by value and call infer_one.  Device code reads the parameters of")
    w("  // the plan's device description, which the model carries by value and whose")
    w("  // buffers stay in place across parameter changes; host code those of the host")
    w("  // description the copies share.")
    w("  __host__ __device__ void infer_one(ponni::SArray<Scalar, num_inputs> const& in,")
    w("                                    ponni::SArray<Scalar, num_outputs>& out) const {")
    w("#if defined(__HIP_DEVICE_COMPILE__)")
    w("    ponni::forward_one_program<Scalar, program>(device_model_.params, in.data(), 1, out.data(), 1);")
    w("#else")
    w("    ponni::forward_one_program<Scalar, program>(state_->host_model.params, in.data(), 1, out.data(), 1);")
    w("#endif")
    w("  }")
    w("  // A trivially copyable handle for kernels that take plain arguments.")
    w("  struct Device {")
    w("    ponni_device_model model;")
    w("    __device__ void infer_one(ponni::SArray<Scalar, num_inputs> const& in,")
    w("                              ponni::SArray<Scalar, num_outputs>& out) const {")
    w("      ponni::forward_one_program<Scalar, program>(model.params, in.data(), 1, out.data(), 1);")
    w("    }")
    w("  };")
    w("  Device device() const { return Device{device_model_}; }")
    w("")
    w(" private:")
    w(f"  static constexpr int num_layers = {len(layers)};")
    w("  static ponni_layer_desc const* descs() {")
    w("    static ponni_layer_desc const d[] = {")
    for l in layers:
        attr = ", ".join(repr(float(a)) for a in l.attr)
        w(f"        {{{l.kind}, {l.n_in}, {l.n_out}, {l.slot}, {l.n_aux}, {l.flags}, {{{attr}}}}},  // {l.label}")
    w("    };")
    w("    return d;")
    w("  }")
    begins = [0]
    for t in tables:
        begins.append(begins[-1] + len(t))
    flat = [x for t in tables for x in t]
    w("  // Layer l's parameter j is gather[begin[l] + j]: a storage index, or -(k + 1) for literals[k].")
    w("  static std::int64_t const* gather() {")
    w("    static std::int64_t const g[] = {")
    for i in range(0, max(len(flat), 1), 16):
        chunk = flat[i:i + 16] if flat else [0]
        w("        " + ", ".join(str(x) for x in chunk) + ",")
    w("    };")
    w("    return g;")
    w("  }")
    w("  static std::int64_t const* begin() {")
    w("    static std::int64_t const b[] = {" + ", ".join(str(x) for x in begins) + "};")
    w("    return b;")
    w("  }")
    w("  static double literal(std::int64_t k) {")
    w("    static double const lit[] = {" + (", ".join(repr(x) for x in literals) if literals else "0.0") + "};")
    w("    return lit[k];")
    w("  }")
    w("")
    w("  std::shared_ptr<ponni_plan_s> make_plan(int dtype) {")
    w("    ponni_plan p = nullptr;")
    w('    ponni::check(ponni_plan_create(descs(), num_layers, dtype, PONNI_PATH_AUTO, &p), "GeneratedModel");')
    w("    return std::shared_ptr<ponni_plan_s>(p, [](ponni_plan q) { ponni_plan_destroy(q); });")
    w("  }")
    w("  void push(ponni_plan plan) {")
    w("    for (int l = 0; l < num_layers; l++) {")
    w("      std::int64_t const n = begin()[l + 1] - begin()[l];")
    w("      if (n == 0) continue;")
    w("      std::vector<Scalar> v(static_cast<std::size_t>(n));")
    w("      for (std::int64_t j = 0; j < n; j++) {")
    w("        std::int64_t const g = gather()[begin()[l] + j];")
    w("        v[j] = static_cast<Scalar>(g >= 0 ? state_->storage[g] : literal(-g - 1));")
    w("      }")
    w('      ponni::check(ponni_plan_set_layer_params(plan, l, v.data(), n), "GeneratedModel parameters");')
    w("    }")
    w("    if (plan != state_->scalar.get()) return;")
    w('    ponni::check(ponni_plan_host_model(plan, &state_->host_model), "GeneratedModel host model");')
    w("    int devices = 0;")
    w("    if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) return;")
    w("    ponni_device_model m{};")
    w('    ponni::check(ponni_plan_device_model(plan, &m), "GeneratedModel device model");')
    w("    // Copies hold device_model_ by value: its buffers must not move once set.")
    w("    if (device_model_.ops != nullptr && (m.ops != device_model_.ops || m.params != device_model_.params))")
    w('      ponni::abort("GeneratedModel device description moved");')
    w("    device_model_ = m;")
    w("  }")
    w("  std::vector<ponni_tensor_spec> cspecs() const {")
    w("    std::vector<ponni_tensor_spec> out;")
    w("    for (auto const& s : weight_specs()) {")
    w("      ponni_tensor_spec t{};")
    w("      t.name = s.name;")
    w("      t.rank = s.rank;")
    w("      for (int k = 0; k < s.rank; k++) t.shape[k] = s.shape[k];")
    w("      t.offset = s.offset;")
    w("      out.push_back(t);")
    w("    }")
    w("    return out;")
    w("  }")
    w("  template <class I, class O>")
    w("  static std::int64_t checked_batch(I const& x, O const& y) {")
    w("    if (x.extent(0) != num_inputs) ponni::abort(\"GeneratedModel input feature extent is incorrect\");")
    w("    if (y.extent(0) != num_outputs) ponni::abort(\"GeneratedModel output feature extent is incorrect\");")
    w("    if (x.extent(1) != y.extent(1)) ponni::abort(\"GeneratedModel batch extents differ\");")
    w("    std::int64_t const b = static_cast<std::int64_t>(x.extent(1));")
    w("    if (b == 0) ponni::abort(\"GeneratedModel::infer_batch requires a nonzero batch size\");")
    w("    return b;")
    w("  }")
    w("  // Launch a generated kernel on the plan's packed parameters.")
    w("  // (PT: the kernel's parameter element type, float, or double for F64 NARROW kernels.)")
    w("  template <class PT, class XT, class YT>")
    w("  void launch(void (*kernel)(PT const*, XT const*, std::int64_t, YT*, std::int64_t, std::int64_t), int threads,")
    w("              int cols, bool persistent, ponni_plan plan, XT const* x, std::int64_t ldx,")
    w("              YT* y, std::int64_t ldy, std::int64_t batch) const {")
    w("    void const* params = nullptr;")
    w('    ponni::check(ponni_plan_device_params(plan, &params), "GeneratedModel parameters");')
    w("    std::int64_t const tiles = (batch + cols - 1) / cols;")
    w("    std::int64_t grid = tiles;")
    w("    if (persistent) {")
    w("      // Resident workgroups of this kernel on the device, found once per kernel.")
    w("      std::int64_t& resident = plan == state_->scalar.get() ? state_->resident[0] : state_->resident[1];")
    w("      if (resident == 0) {")
    w("        int dev = 0, cus = 0, per = 0;")
    w("        (void)hipGetDevice(&dev);")
    w("        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);")
    w("        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, 0);")
    w("        resident = std::int64_t(std::max(cus, 1)) * std::max(per, 1);")
    w("      }")
    w("      grid = std::min<std::int64_t>(tiles, resident);")
    w("    }")
    w("    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(threads), 0, state_->stream,")
    w("                       static_cast<PT const*>(params), x, ldx, y, ldy, batch);")
    w("    hipError_t const e = hipGetLastError();")
    w('    if (e != hipSuccess) ponni::abort(std::string("GeneratedModel kernel launch: ") + hipGetErrorString(e));')
    w("  }")
    w("  // Row-strided [rows, cols] -> [rows, cols] conversion of n elements.")
    w("  template <class From, class To>")
    w("  static __global__ void convert_rows(From const* __restrict__ src, std::int64_t lds, To* __restrict__ dst,")
    w("                                      std::int64_t ldd, std::int64_t n, std::int64_t cols) {")
    w("    std::int64_t const i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;")
    w("    if (i >= n) return;")
    w("    std::int64_t const r = i / cols, c = i % cols;")
    w("    dst[r * ldd + c] = static_cast<To>(static_cast<float>(src[r * lds + c]));")
    w("  }")
    w("  void half_buffers(std::int64_t batch) const {")
    w("    if (batch <= state_->half_capacity) return;")
    w("    if (state_->hx) (void)hipFree(state_->hx);")
    w("    if (state_->hy) (void)hipFree(state_->hy);")
    w('    if (hipMalloc(&state_->hx, sizeof(_Float16) * num_inputs * batch) != hipSuccess) ponni::abort("hipMalloc");')
    w('    if (hipMalloc(&state_->hy, sizeof(_Float16) * num_outputs * batch) != hipSuccess) ponni::abort("hipMalloc");')
    w("    state_->half_capacity = batch;")
    w("  }")
    w("")
    w("  struct State {")
    w("    hipStream_t stream = nullptr;")
    w("    std::vector<double> storage;")
    w("    bool loaded = false;")
    w("    std::shared_ptr<ponni_plan_s> scalar, half;")
    w("    ponni_device_model host_model{};")
    w("    _Float16* hx = nullptr;")
    w("    _Float16* hy = nullptr;")
    w("    std::int64_t half_capacity = 0;")
    w("    std::int64_t resident[2] = {0, 0};")
    w("    State() = default;")
    w("    State(State const&) = delete;")
    w("    State& operator=(State const&) = delete;")
    w("    ~State() {")
    w("      if (hx) (void)hipFree(hx);")
    w("      if (hy) (void)hipFree(hy);")
    w("    }")
    w("  };")
    w("  // First member: device code reads it at the same offset host code wrote it.")
    w("  ponni_device_model device_model_{};")
    w("  std::shared_ptr<State> state_;")
    w("};")
    w("")
    w(ns_close)
    text = "\n".join(o) + "\n"
    with open(path, "w") as f:
        f.write(text)
    return text
