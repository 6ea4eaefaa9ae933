// ponni.h -- header-only C++17 facade of PONNI's template API over
// libponni_hip.so (include/ponni_hip.h).
//
// It keeps the reference's host-side surface so application code drops in:
//   - layer templates            src/layers/*.h (Matvec, Bias, Relu, ..., Save_State,
//                                Binop_Add, Binop_Concatenate, Binop_Projection_Add)
//   - create_inference_model     src/ponni_create_model.h:40-98 (plus the
//                                _single / _double / _half / _bhalf_precision factories)
//   - Inference                  src/ponni_Inference.h: forward_batch_parallel(in[, out]),
//                                validate, print, reallocate_internal_state,
//                                internal_state_capacity, get_layer<I>, get/set
//                                trainable parameters, save/load_weights,
//                                weight_schema_fingerprint
//   - the View contract          src/utils/ponni_kokkos_utils.h:11-25: rank-2
//                                LayoutRight [features, batch] device arrays
//   - .ponni files               src/utils/ponni_safetensors.h via ponni/ponni_file.h,
//                                load_ponni_tensor and the View copies of
//                                src/utils/ponni_view_ops.h
//
// What changes underneath: the per-sample Kokkos RangePolicy executor is
// replaced by one call of ponni_forward(), which runs a gfx950 kernel chosen
// (and, for wide models, generated) for the whole layer chain.  Models bound
// to the host execution space (create_inference_model(Host(), HostSpace(),
// ...)) run on host threads through ponni_forward_host instead, on host Views.  Layers hold
// their parameters on the host; the plan owns the packed device copy and is
// refreshed whenever parameters change.  A View here is any type with
// data(), extent(0), extent(1), stride(0) and a LayoutRight array_layout:
// ponni::View below, or a Kokkos::View with Kokkos::LayoutRight.
//
// Build: hipcc -std=c++17 -I<repo>/include -I<repo>/ponni_amd/include app.cpp
//        -L<repo>/ponni_amd -lponni_hip
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <ctime>
#include <iomanip>
#include <iostream>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <tuple>
#include <type_traits>
#include <utility>
#include <vector>

#include "ponni/device.h"
#include "ponni/ponni_file.h"
#include "ponni_hip.h"

namespace ponni {

// ---- errors ---------------------------------------------------------------------

// Print and abort, as Kokkos::abort does for the reference's shape errors.
[[noreturn]] inline void abort(std::string const& message) {
  std::fprintf(stderr, "%s\n", message.c_str());
  std::fflush(stderr);
  std::abort();
}

inline void check(int status, char const* what = "ponni") {
  if (status != PONNI_OK) abort(std::string(what) + ": " + ponni_last_error());
}

// ---- scalar types -------------------------------------------------------------------

// 16-bit storage types of the half / bfloat16 models (Kokkos::Experimental::
// half_t / bhalf_t).  Host conversions round to nearest even.
struct half_t {
  std::uint16_t bits = 0;
  half_t() = default;
  half_t(float f) : bits(from_float(f)) {}
  operator float() const { return to_float(bits); }
  static std::uint16_t from_float(float f) {
    std::uint32_t x;
    std::memcpy(&x, &f, 4);
    std::uint32_t const sign = (x >> 16) & 0x8000u;
    std::uint32_t const ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return static_cast<std::uint16_t>(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return static_cast<std::uint16_t>(sign | 0x7c00u);  // rounds past 65504
    if (ax < 0x38800000u) {  // subnormal or zero: quantum 2^-24
      float const a = std::fabs(f) * 16777216.0f;
      return static_cast<std::uint16_t>(sign | static_cast<std::uint32_t>(std::nearbyint(a)));
    }
    std::uint32_t const lsb = (ax >> 13) & 1u;
    std::uint32_t const r = ax + 0xfffu + lsb;
    return static_cast<std::uint16_t>(sign | ((r - 0x38000000u) >> 13));
  }
  static float to_float(std::uint16_t h) {
    std::uint32_t const sign = static_cast<std::uint32_t>(h & 0x8000u) << 16;
    std::uint32_t const e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    float out;
    if (e == 0) {
      out = std::ldexp(static_cast<float>(m), -24);
      return sign ? -out : out;
    }
    std::uint32_t const x = sign | (e == 31 ? 0x7f800000u | (m << 13) : ((e + 112u) << 23) | (m << 13));
    std::memcpy(&out, &x, 4);
    return out;
  }
};

struct bhalf_t {
  std::uint16_t bits = 0;
  bhalf_t() = default;
  bhalf_t(float f) {
    std::uint32_t x;
    std::memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) {
      bits = static_cast<std::uint16_t>((x >> 16) | 0x40u);
    } else {
      x += 0x7fffu + ((x >> 16) & 1u);
      bits = static_cast<std::uint16_t>(x >> 16);
    }
  }
  operator float() const {
    std::uint32_t const x = static_cast<std::uint32_t>(bits) << 16;
    float f;
    std::memcpy(&f, &x, 4);
    return f;
  }
};

template <class real> constexpr int dtype_of() {
  if constexpr (std::is_same_v<real, double>) return PONNI_F64;
  else if constexpr (std::is_same_v<real, half_t>) return PONNI_F16;
  else if constexpr (std::is_same_v<real, bhalf_t>) return PONNI_BF16;
  else {
    static_assert(std::is_same_v<real, float>, "real must be float, double, half_t or bhalf_t");
    return PONNI_F32;
  }
}

// ---- views ---------------------------------------------------------------------------

struct LayoutRight {};

// Trivially copyable handle of a View for device code (kernel arguments,
// lambda captures): the same accessors, no ownership.
template <class T>
struct DeviceView {
  using value_type = T;
  using array_layout = LayoutRight;
  static constexpr int rank = 2;
  T* data_;
  std::int64_t rows_, cols_, ld_;
  __host__ __device__ T* data() const { return data_; }
  __host__ __device__ std::int64_t extent(int d) const { return d == 0 ? rows_ : cols_; }
  __host__ __device__ std::int64_t stride(int d) const { return d == 0 ? ld_ : 1; }
  __host__ __device__ T& operator()(std::int64_t r, std::int64_t c) const { return data_[r * ld_ + c]; }
};

// ---- execution and memory spaces ---------------------------------------------------------
// The reference selects where a model runs with a Kokkos execution space and
// memory space (src/ponni_create_model.h:21-90).  Here:
//   HIP  (memory HIPSpace)   the GPU; holds the stream the model launches on
//                            (the default execution space);
//   Host (memory HostSpace)  the calling host, `threads` host threads (0: one
//                            per hardware thread) through the library's host
//                            executor (ponni_forward_host); the default host
//                            execution space.
struct HostSpace {};
struct HIPSpace {};
struct HIP {
  using memory_space = HIPSpace;
  hipStream_t stream = nullptr;
  HIP() = default;
  explicit HIP(hipStream_t s) : stream(s) {}
};
struct Host {
  using memory_space = HostSpace;
  int threads = 0;
  Host() = default;
  explicit Host(int n) : threads(n) {}
};
using DefaultExecutionSpace = HIP;
using DefaultHostExecutionSpace = Host;

template <class E> struct is_execution_space : std::false_type {};
template <> struct is_execution_space<HIP> : std::true_type {};
template <> struct is_execution_space<Host> : std::true_type {};
template <class E> inline constexpr bool is_execution_space_v = is_execution_space<std::decay_t<E>>::value;
template <class M> struct is_memory_space : std::false_type {};
template <> struct is_memory_space<HIPSpace> : std::true_type {};
template <> struct is_memory_space<HostSpace> : std::true_type {};
template <class M> inline constexpr bool is_memory_space_v = is_memory_space<std::decay_t<M>>::value;

// The memory space a view type declares (HIPSpace when it declares none: a
// device pointer is what forward_batch_parallel has always taken).
template <class V, class = void> struct view_memory_space { using type = HIPSpace; };
template <class V> struct view_memory_space<V, std::void_t<typename V::memory_space>> {
  using type = std::conditional_t<std::is_same_v<typename V::memory_space, HostSpace>, HostSpace, HIPSpace>;
};

// A rank-2 LayoutRight [rows, cols] array in device memory (HIPSpace, the
// default) or host memory (HostSpace); element (r, c) at
// data()[r * stride(0) + c].  Copies share the allocation (as Kokkos::View).
template <class T, class Space = HIPSpace>
class View {
  static_assert(is_memory_space_v<Space>, "ponni::View memory space must be HIPSpace or HostSpace");
  static constexpr bool on_host = std::is_same_v<Space, HostSpace>;

 public:
  using value_type = T;
  using non_const_value_type = std::remove_const_t<T>;
  using array_layout = LayoutRight;
  using memory_space = Space;
  static constexpr int rank = 2;

  View() = default;
  View(std::string label, std::int64_t rows, std::int64_t cols, bool zero = true)
      : label_(std::move(label)), rows_(rows), cols_(cols), ld_(cols) {
    if (rows < 0 || cols < 0) abort("ponni::View extents must be nonnegative");
    if (rows * cols > 0) {
      std::size_t const bytes = sizeof(T) * static_cast<std::size_t>(rows * cols);
      void* p = nullptr;
      if constexpr (on_host) {
        p = std::calloc(static_cast<std::size_t>(rows * cols), sizeof(T));
        if (p == nullptr) abort("ponni::View host allocation failed");
        owner_ = std::shared_ptr<void>(p, [](void* q) { std::free(q); });
      } else {
        check_hip(hipMalloc(&p, bytes), "hipMalloc");
        if (zero) check_hip(hipMemset(p, 0, bytes), "hipMemset");
        owner_ = std::shared_ptr<void>(p, [](void* q) { (void)hipFree(q); });
      }
      data_ = static_cast<T*>(p);
    }
  }
  // Wrap caller-owned memory of this space (no ownership).
  static View wrap(T* data, std::int64_t rows, std::int64_t cols, std::int64_t ld) {
    View v;
    v.data_ = data;
    v.rows_ = rows;
    v.cols_ = cols;
    v.ld_ = ld;
    return v;
  }
  // Columns [c0, c1) of this view (a LayoutRight subview with stride(0) > extent(1)).
  View columns(std::int64_t c0, std::int64_t c1) const {
    View v = *this;
    v.data_ = data_ + c0;
    v.cols_ = c1 - c0;
    return v;
  }
  // The same contiguous elements as a [rows, cols] view (shares the allocation).
  View reshape(std::int64_t rows, std::int64_t cols) const {
    if (rows * cols != size() || (rows_ > 1 && ld_ != cols_))
      abort("ponni::View::reshape needs a contiguous view of the same size");
    View v = *this;
    v.rows_ = rows;
    v.cols_ = cols;
    v.ld_ = cols;
    return v;
  }

  __host__ __device__ T* data() const { return data_; }
  __host__ __device__ std::int64_t extent(int d) const { return d == 0 ? rows_ : cols_; }
  __host__ __device__ std::int64_t stride(int d) const { return d == 0 ? ld_ : 1; }
  __host__ __device__ T& operator()(std::int64_t r, std::int64_t c) const { return data_[r * ld_ + c]; }
  DeviceView<T> device() const { return DeviceView<T>{data_, rows_, cols_, ld_}; }
  std::int64_t size() const { return rows_ * cols_; }
  bool is_allocated() const { return data_ != nullptr; }
  std::string const& label() const { return label_; }

  // Copies from / to a row-major [rows, cols] host array.
  void copy_from_host(std::vector<non_const_value_type> const& h) const {
    if (static_cast<std::int64_t>(h.size()) != size()) abort("ponni::View::copy_from_host size mismatch");
    if (size() == 0) return;
    if constexpr (on_host) {
      for (std::int64_t r = 0; r < rows_; r++)
        std::memcpy(const_cast<non_const_value_type*>(data_) + r * ld_, h.data() + r * cols_, sizeof(T) * cols_);
    } else {
      check_hip(hipMemcpy2D(data_, sizeof(T) * ld_, h.data(), sizeof(T) * cols_, sizeof(T) * cols_, rows_,
                            hipMemcpyHostToDevice),
                "hipMemcpy2D");
    }
  }
  std::vector<non_const_value_type> copy_to_host() const {
    std::vector<non_const_value_type> h(static_cast<std::size_t>(size()));
    if (size() == 0) return h;
    if constexpr (on_host) {
      for (std::int64_t r = 0; r < rows_; r++) std::memcpy(h.data() + r * cols_, data_ + r * ld_, sizeof(T) * cols_);
    } else {
      check_hip(hipMemcpy2D(h.data(), sizeof(T) * cols_, data_, sizeof(T) * ld_, sizeof(T) * cols_, rows_,
                            hipMemcpyDeviceToHost),
                "hipMemcpy2D");
    }
    return h;
  }

 private:
  static void check_hip(hipError_t e, char const* what) {
    if (e != hipSuccess) abort(std::string(what) + ": " + hipGetErrorString(e));
  }
  std::string label_;
  std::shared_ptr<void> owner_;
  T* data_ = nullptr;
  std::int64_t rows_ = 0, cols_ = 0, ld_ = 0;
};

// Fixed-size per-thread array (ponni::SArray of the reference, used by the
// in-kernel SArray form of forward_batch_parallel_in_kernel).
template <class T, int N>
struct SArray {
  T v[N > 0 ? N : 1];
  __host__ __device__ T& operator()(int i) { return v[i]; }
  __host__ __device__ T const& operator()(int i) const { return v[i]; }
  __host__ __device__ T& operator[](int i) { return v[i]; }
  __host__ __device__ T const& operator[](int i) const { return v[i]; }
  __host__ __device__ T* data() { return v; }
  __host__ __device__ T const* data() const { return v; }
  static constexpr int size() { return N; }
};

// LayoutRight check of the View contract (ponni_kokkos_utils.h:11-25).
template <class V, class = void>
struct is_layout_right_view : std::false_type {};
template <class V>
struct is_layout_right_view<V, std::void_t<typename V::array_layout>>
    : std::bool_constant<std::is_same_v<typename V::array_layout, LayoutRight>
#ifdef KOKKOS_VERSION
                         || std::is_same_v<typename V::array_layout, Kokkos::LayoutRight>
#endif
                         > {
};
template <class V>
inline constexpr bool is_layout_right_view_v = is_layout_right_view<std::decay_t<V>>::value;

template <class... Views>
constexpr void require_layout_right_views() {
  static_assert((is_layout_right_view_v<Views> && ...), "PONNI Views must use LayoutRight");
}

// ---- host arrays and initializers ------------------------------------------------------

// A host row-major matrix used to hand weights to layer constructors.
template <class real>
struct Matrix {
  int rows = 0, cols = 0;
  std::vector<real> values;
  Matrix() = default;
  Matrix(int r, int c, real fill = real(0)) : rows(r), cols(c), values(static_cast<std::size_t>(r) * c, fill) {}
  Matrix(int r, int c, std::vector<real> v) : rows(r), cols(c), values(std::move(v)) {
    if (static_cast<std::int64_t>(values.size()) != static_cast<std::int64_t>(r) * c) abort("ponni::Matrix size mismatch");
  }
  real& operator()(int i, int j) { return values[static_cast<std::size_t>(i) * cols + j]; }
  real operator()(int i, int j) const { return values[static_cast<std::size_t>(i) * cols + j]; }
  int extent(int d) const { return d == 0 ? rows : cols; }
};

namespace init_detail {
inline std::uint64_t splitmix64(std::uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
inline std::uint64_t effective_seed(std::uint64_t seed) {
  return seed == 0 ? static_cast<std::uint64_t>(std::time(nullptr)) : seed;
}
// Uniform [0, 1) of element i of a fill (53 random bits).
inline double unit(std::uint64_t seed, std::uint64_t i) {
  return static_cast<double>(splitmix64(seed ^ splitmix64(i + 1)) >> 11) * (1.0 / 9007199254740992.0);
}
inline double normal(std::uint64_t seed, std::uint64_t i) {
  double const u1 = 1.0 - unit(seed, 2 * i), u2 = unit(seed, 2 * i + 1);
  return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}
}  // namespace init_detail

// Initializers of src/initializers/ponni_initializer.h (same parameters and
// fan conventions: a [n_in, n_out] weight has fan_in = n_in, fan_out = n_out).
// The random streams are this library's own (splitmix64 per element); the
// reference's Kokkos XorShift streams are not reproduced.
template <class real>
struct Initializer_Random_Uniform {
  double lb = -0.05, ub = 0.05;
  std::uint64_t seed = 0;
  Initializer_Random_Uniform(real lb_ = real(-0.05), real ub_ = real(0.05), std::uint64_t seed_ = 0)
      : lb(lb_), ub(ub_), seed(seed_) {
    if (!(lb <= ub)) throw std::invalid_argument("Initializer_Random_Uniform requires lower bound <= upper bound");
  }
  void fill(std::vector<double>& a, int, int) const {
    std::uint64_t const s = init_detail::effective_seed(seed);
    for (std::size_t i = 0; i < a.size(); i++) a[i] = lb + (ub - lb) * init_detail::unit(s, i);
  }
};
template <class real>
struct Initializer_Random_Normal {
  double mean = 0, stdev = 1;
  std::uint64_t seed = 0;
  Initializer_Random_Normal(real m = real(0), real s = real(1), std::uint64_t sd = 0) : mean(m), stdev(s), seed(sd) {}
  void fill(std::vector<double>& a, int, int) const {
    std::uint64_t const s = init_detail::effective_seed(seed);
    for (std::size_t i = 0; i < a.size(); i++) a[i] = mean + stdev * init_detail::normal(s, i);
  }
};
template <class real>
struct Initializer_Constant {
  double value = 0;
  explicit Initializer_Constant(real v = real(0)) : value(v) {}
  void fill(std::vector<double>& a, int, int) const {
    for (double& v : a) v = value;
  }
};
template <class real> struct Initializer_Zeros : Initializer_Constant<real> { Initializer_Zeros() : Initializer_Constant<real>(real(0)) {} };
template <class real> struct Initializer_Ones : Initializer_Constant<real> { Initializer_Ones() : Initializer_Constant<real>(real(1)) {} };
struct Initializer_Xavier_Uniform {
  std::uint64_t seed = 0;
  explicit Initializer_Xavier_Uniform(std::uint64_t s = 0) : seed(s) {}
  void fill(std::vector<double>& a, int fan_in, int fan_out) const {
    double const lim = std::sqrt(6.0 / (fan_in + fan_out));
    Initializer_Random_Uniform<double>(-lim, lim, seed).fill(a, fan_in, fan_out);
  }
};
struct Initializer_Xavier_Normal {
  std::uint64_t seed = 0;
  explicit Initializer_Xavier_Normal(std::uint64_t s = 0) : seed(s) {}
  void fill(std::vector<double>& a, int fan_in, int fan_out) const {
    Initializer_Random_Normal<double>(0.0, std::sqrt(2.0 / (fan_in + fan_out)), seed).fill(a, fan_in, fan_out);
  }
};
struct Initializer_He_Uniform {
  std::uint64_t seed = 0;
  explicit Initializer_He_Uniform(std::uint64_t s = 0) : seed(s) {}
  void fill(std::vector<double>& a, int fan_in, int fan_out) const {
    double const lim = std::sqrt(6.0 / fan_in);
    Initializer_Random_Uniform<double>(-lim, lim, seed).fill(a, fan_in, fan_out);
  }
};
struct Initializer_He_Normal {
  std::uint64_t seed = 0;
  explicit Initializer_He_Normal(std::uint64_t s = 0) : seed(s) {}
  void fill(std::vector<double>& a, int fan_in, int fan_out) const {
    Initializer_Random_Normal<double>(0.0, std::sqrt(2.0 / fan_in), seed).fill(a, fan_in, fan_out);
  }
};

// ---- layer classification (ponni_LayerTraits.h:10-61) ------------------------------------

// Whether a layer may be fused with its neighbours.  A layer without a
// static constexpr `fusion_kind` is a barrier.  Built-in layers declare it;
// a user layer (the plugin contract) opts in the same way and then provides
//   dense:     static real compute_output(input, int feature, int batch, Params const&)
//   pointwise: static real apply_fused(value, int feature, Params const&)
//              (or apply(value, Params const&), or apply(value))
//   barrier:   static void compute_all_outputs(input, output, int batch, Params const&)
//              (binop layers: compute_all_outputs(input, saved, output, batch, params))
// as __host__ __device__ functions, a device-copyable nested `Params`, a
// `params` member, get_num_inputs() / get_num_outputs(), and the flags
// overwrite_input / save / binop (with `index` = ISAVE) of the reference.
enum class LayerFusionKind { barrier, dense, pointwise };

template <class Layer, class = void>
struct LayerTraits {
  static constexpr LayerFusionKind fusion_kind = LayerFusionKind::barrier;
};
template <class Layer>
struct LayerTraits<Layer, std::void_t<decltype(Layer::fusion_kind)>> {
  static constexpr LayerFusionKind fusion_kind = Layer::fusion_kind;
};
template <class Layer>
inline constexpr bool is_dense_layer_v = LayerTraits<Layer>::fusion_kind == LayerFusionKind::dense;
template <class Layer>
inline constexpr bool is_pointwise_layer_v = LayerTraits<Layer>::fusion_kind == LayerFusionKind::pointwise;

namespace detail {
template <class L, class R, class P, class = void>
struct has_apply_fused : std::false_type {};
template <class L, class R, class P>
struct has_apply_fused<L, R, P, std::void_t<decltype(L::apply_fused(std::declval<R>(), 0, std::declval<P const&>()))>>
    : std::true_type {};
template <class L, class R, class P, class = void>
struct has_apply_p : std::false_type {};
template <class L, class R, class P>
struct has_apply_p<L, R, P, std::void_t<decltype(L::apply(std::declval<R>(), std::declval<P const&>()))>>
    : std::true_type {};
}  // namespace detail

// One pointwise layer on one value (the three forms of ponni_LayerTraits.h:49-61).
template <class Layer, class Real>
__host__ __device__ inline Real apply_fused_layer(Real value, int feature, typename Layer::Params const& params) {
  if constexpr (detail::has_apply_fused<Layer, Real, typename Layer::Params>::value) {
    return Layer::apply_fused(value, feature, params);
  } else if constexpr (detail::has_apply_p<Layer, Real, typename Layer::Params>::value) {
    return Layer::apply(value, params);
  } else {
    return Layer::apply(value);
  }
}

// ---- layers -----------------------------------------------------------------------------

namespace detail {

// Common state of every built-in layer: the C-ABI descriptor and the host
// master copy of its parameters in the layer's own order.
struct LayerCore {
  ponni_layer_desc desc{};
  std::vector<double> params;
  bool trainable = false;
  char const* label = "";
  std::uint64_t version = 0;  // bumped on every parameter change

  int get_num_inputs() const { return desc.n_in; }
  int get_num_outputs() const { return desc.n_out; }
  char const* get_label() const { return label; }
  int get_num_trainable_parameters() const { return trainable ? static_cast<int>(params.size()) : 0; }

  // Consume the first get_num_trainable_parameters() values (ponni_Matvec.h:103-109).
  template <class Vec>
  void set_trainable_parameters(Vec const& in) {
    if (!trainable) return;
    if (static_cast<std::int64_t>(in.size()) < static_cast<std::int64_t>(params.size()))
      abort(std::string("ERROR: ") + label + " trainable input too small");
    for (std::size_t i = 0; i < params.size(); i++) params[i] = static_cast<double>(in[i]);
    version++;
  }
  std::vector<double> get_trainable_parameters() const { return trainable ? params : std::vector<double>(); }
  // Call after writing `params` directly.
  void mark_modified() { version++; }
};

inline ponni_layer_desc make_desc(int kind, int n_in, int n_out, int slot = 0, int n_aux = 0, int flags = 0,
                                  double a0 = 0, double a1 = 0, double a2 = 0) {
  ponni_layer_desc d{};
  d.kind = kind;
  d.n_in = n_in;
  d.n_out = n_out;
  d.slot = slot;
  d.n_aux = n_aux;
  d.flags = flags;
  d.attr[0] = a0;
  d.attr[1] = a1;
  d.attr[2] = a2;
  return d;
}

template <class M>
std::vector<double> flatten(M const& m) {
  std::vector<double> v(static_cast<std::size_t>(m.extent(0)) * m.extent(1));
  for (int i = 0; i < static_cast<int>(m.extent(0)); i++)
    for (int j = 0; j < static_cast<int>(m.extent(1)); j++)
      v[static_cast<std::size_t>(i) * m.extent(1) + j] = static_cast<double>(m(i, j));
  return v;
}

template <class V>
std::vector<double> flatten1(V const& v) {
  std::vector<double> out(v.size());
  for (std::size_t i = 0; i < out.size(); i++) out[i] = static_cast<double>(v[i]);
  return out;
}

// ponni::View arguments (device or host memory) are read through a host copy.
template <class T, class Space>
std::vector<double> flatten(View<T, Space> const& m) {
  auto const h = m.copy_to_host();
  return std::vector<double>(h.begin(), h.end());
}
template <class T, class Space>
std::vector<double> flatten1(View<T, Space> const& v) {
  return detail::flatten(v);
}

}  // namespace detail

// Dense layer, W [n_in, n_out] (ponni_Matvec.h).  Constructors: (num_inputs,
// num_outputs, trainable, initializer) or (weights [n_in, n_out], trainable).
template <class real = float, int N_IN = 1, int N_OUT = 1>
struct Matvec : detail::LayerCore {
  static constexpr LayerFusionKind fusion_kind = LayerFusionKind::dense;
  static constexpr int INPUT_SIZE = N_IN, OUTPUT_SIZE = N_OUT;
  Matvec() = default;
  template <class INIT = Initializer_Random_Uniform<real>>
  Matvec(int num_inputs, int num_outputs, bool trainable_ = true, INIT init = INIT()) {
    std::vector<double> w(static_cast<std::size_t>(num_inputs) * num_outputs);
    init.fill(w, num_inputs, num_outputs);
    setup(num_inputs, num_outputs, std::move(w), trainable_);
  }
  template <class M, class = decltype(std::declval<M const&>()(0, 0))>
  explicit Matvec(M const& weights, bool trainable_ = true) {
    setup(static_cast<int>(weights.extent(0)), static_cast<int>(weights.extent(1)), detail::flatten(weights),
          trainable_);
  }
  void setup(int n_in, int n_out, std::vector<double> w, bool t) {
    if (n_in <= 0 || n_out <= 0) abort("ERROR: Matvec weights dimensions must be nonzero");
    desc = detail::make_desc(PONNI_LAYER_MATVEC, n_in, n_out);
    params = std::move(w);
    trainable = t;
    label = "Matvec";
  }
  // W(k, j) of the [n_in, n_out] weights.
  double weight(int k, int j) const { return params[static_cast<std::size_t>(k) * desc.n_out + j]; }
  void validate() const {
    if (desc.n_in <= 0 || desc.n_out <= 0) abort("ERROR: Matvec weights dimensions must be nonzero");
  }
};

// Bias (ponni_Bias.h): (num_inputs, trainable, initializer) or (weights, trainable).
template <class real = float, int N = 1>
struct Bias : detail::LayerCore {
  static constexpr LayerFusionKind fusion_kind = LayerFusionKind::pointwise;
  static constexpr int INPUT_SIZE = N, OUTPUT_SIZE = N;
  Bias() = default;
  template <class INIT = Initializer_Random_Uniform<real>>
  Bias(int num_inputs, bool trainable_ = true, INIT init = INIT()) {
    std::vector<double> b(static_cast<std::size_t>(num_inputs));
    init.fill(b, num_inputs, num_inputs);
    setup(std::move(b), trainable_);
  }
  template <class V, class = decltype(std::declval<V const&>()[0]), class = decltype(std::declval<V const&>().size())>
  explicit Bias(V const& weights, bool trainable_ = true) {
    setup(detail::flatten1(weights), trainable_);
  }
  // A [1, n] or [n, 1] View (load_ponni_tensor<1>), in any memory space.
  template <class T, class Space>
  explicit Bias(View<T, Space> const& weights, bool trainable_ = true) {
    setup(detail::flatten1(weights), trainable_);
  }
  void setup(std::vector<double> b, bool t) {
    int const n = static_cast<int>(b.size());
    desc = detail::make_desc(PONNI_LAYER_BIAS, n, n);
    params = std::move(b);
    trainable = t;
    label = "Bias";
  }
  void validate() const {
    if (desc.n_in <= 0) abort("ERROR: Bias weights dimension must be nonzero");
  }
};

namespace detail {
// Parameter-free pointwise / barrier layers share this shape.
template <int KIND>
struct Simple : LayerCore {
  static constexpr LayerFusionKind fusion_kind =
      (KIND == PONNI_LAYER_SOFTMAX || KIND == PONNI_LAYER_LOG_SOFTMAX || KIND == PONNI_LAYER_MIN_MAX_NORM)
          ? LayerFusionKind::barrier
          : LayerFusionKind::pointwise;
  Simple() = default;
  Simple(int n, char const* lbl, int flags = 0, double a0 = 0, double a1 = 0, double a2 = 0) {
    desc = make_desc(KIND, n, n, 0, 0, flags, a0, a1, a2);
    label = lbl;
  }
  void validate() const {
    if (desc.n_in <= 0) abort(std::string("ERROR: ") + label + " num_inputs must be > 0");
  }
};
}  // namespace detail

template <class real = float, int N = 1>
struct Relu : detail::Simple<PONNI_LAYER_RELU> {
  static constexpr int INPUT_SIZE = N, OUTPUT_SIZE = N;
  Relu() = default;
  explicit Relu(int n) : Simple(n, "ReLU") {}
};
template <class real = float, int N = 1>
struct LeakyRelu : detail::Simple<PONNI_LAYER_LEAKY_RELU> {
  LeakyRelu() = default;
  explicit LeakyRelu(int n, real negative_slope = real(0.01))
      : Simple(n, "LeakyReLU", 0, static_cast<double>(negative_slope)) {}
};
template <class real = float, int N = 1>
struct Elu : detail::Simple<PONNI_LAYER_ELU> {
  Elu() = default;
  explicit Elu(int n, real alpha = real(1)) : Simple(n, "ELU", 0, static_cast<double>(alpha)) {
    if (!(static_cast<double>(alpha) > 0)) abort("ERROR: ELU alpha must be > 0");
  }
};
template <class real = float, int N = 1>
struct Selu : detail::Simple<PONNI_LAYER_SELU> {
  Selu() = default;
  explicit Selu(int n) : Simple(n, "SELU") {}
};
template <class real = float, int N = 1>
struct Gelu : detail::Simple<PONNI_LAYER_GELU> {
  Gelu() = default;
  explicit Gelu(int n, bool approximate = false)
      : Simple(n, "GELU", approximate ? PONNI_FLAG_GELU_APPROXIMATE : 0) {}
};
template <class real = float, int N = 1>
struct Silu : detail::Simple<PONNI_LAYER_SILU> {
  Silu() = default;
  explicit Silu(int n) : Simple(n, "SiLU") {}
};
template <class real = float, int N = 1>
struct Sigmoid : detail::Simple<PONNI_LAYER_SIGMOID> {
  Sigmoid() = default;
  explicit Sigmoid(int n) : Simple(n, "Sigmoid") {}
};
template <class real = float, int N = 1>
struct Tanh : detail::Simple<PONNI_LAYER_TANH> {
  Tanh() = default;
  explicit Tanh(int n) : Simple(n, "Tanh") {}
};
template <class real = float, int N = 1>
struct Softplus : detail::Simple<PONNI_LAYER_SOFTPLUS> {
  Softplus() = default;
  explicit Softplus(int n, real beta = real(1)) : Simple(n, "Softplus", 0, static_cast<double>(beta)) {
    if (!(static_cast<double>(beta) > 0)) abort("ERROR: Softplus beta must be > 0");
  }
};
template <class real = float, int N = 1>
struct HardSigmoid : detail::Simple<PONNI_LAYER_HARD_SIGMOID> {
  HardSigmoid() = default;
  explicit HardSigmoid(int n, real alpha = real(0.2), real beta = real(0.5))
      : Simple(n, "HardSigmoid", 0, static_cast<double>(alpha), static_cast<double>(beta)) {}
};
template <class real = float, int N = 1>
struct HardSwish : detail::Simple<PONNI_LAYER_HARD_SWISH> {
  HardSwish() = default;
  explicit HardSwish(int n) : Simple(n, "HardSwish") {}
};
template <class real = float, int N = 1>
struct Mish : detail::Simple<PONNI_LAYER_MISH> {
  Mish() = default;
  explicit Mish(int n) : Simple(n, "Mish") {}
};
template <class real = float, int N = 1>
struct Softmax : detail::Simple<PONNI_LAYER_SOFTMAX> {
  Softmax() = default;
  explicit Softmax(int n) : Simple(n, "Softmax") {}
};
template <class real = float, int N = 1>
struct LogSoftmax : detail::Simple<PONNI_LAYER_LOG_SOFTMAX> {
  LogSoftmax() = default;
  explicit LogSoftmax(int n) : Simple(n, "LogSoftmax") {}
};
template <class real = float, int N = 1>
struct MinMaxNorm : detail::Simple<PONNI_LAYER_MIN_MAX_NORM> {
  MinMaxNorm() = default;
  explicit MinMaxNorm(int n, real out_min = real(0), real out_max = real(1), real epsilon = real(1e-12))
      : Simple(n, "MinMaxNorm", 0, static_cast<double>(out_min), static_cast<double>(out_max),
               static_cast<double>(epsilon)) {}
};

// LayerNorm (ponni_LayerNorm.h): gamma = 1, beta = 0 by default; trainable [gamma; beta].
template <class real = float, int N = 1>
struct LayerNorm : detail::LayerCore {
  LayerNorm() = default;
  explicit LayerNorm(int n, real epsilon = real(1e-5), bool trainable_ = true) {
    std::vector<double> p(2 * static_cast<std::size_t>(n), 0.0);
    for (int i = 0; i < n; i++) p[i] = 1.0;
    setup(n, std::move(p), epsilon, trainable_);
  }
  template <class V, class = decltype(std::declval<V const&>()[0])>
  LayerNorm(V const& gamma, V const& beta, real epsilon = real(1e-5), bool trainable_ = true) {
    if (gamma.size() != beta.size()) abort("ERROR: LayerNorm gamma/beta sizes differ");
    std::vector<double> p = detail::flatten1(gamma), b = detail::flatten1(beta);
    p.insert(p.end(), b.begin(), b.end());
    setup(static_cast<int>(gamma.size()), std::move(p), epsilon, trainable_);
  }
  template <class T, class Space>
  LayerNorm(View<T, Space> const& gamma, View<T, Space> const& beta, real epsilon = real(1e-5),
            bool trainable_ = true) {
    if (gamma.size() != beta.size()) abort("ERROR: LayerNorm gamma/beta sizes differ");
    std::vector<double> p = detail::flatten1(gamma), b = detail::flatten1(beta);
    p.insert(p.end(), b.begin(), b.end());
    setup(static_cast<int>(gamma.size()), std::move(p), epsilon, trainable_);
  }
  void setup(int n, std::vector<double> p, real epsilon, bool t) {
    if (!(static_cast<double>(epsilon) > 0)) abort("ERROR: LayerNorm epsilon must be > 0");
    desc = detail::make_desc(PONNI_LAYER_LAYER_NORM, n, n, 0, 0, 0, static_cast<double>(epsilon));
    params = std::move(p);
    trainable = t;
    label = "LayerNorm";
  }
  void validate() const {}
};

// Residual plumbing (ponni_Save_State.h, ponni_Binop_*.h).  ISAVE selects the
// saved-state slot, as the reference's first template argument.
template <int ISAVE, class real = float, int N = 1>
struct Save_State : detail::LayerCore {
  static constexpr bool save = true, binop = false;
  static constexpr int index = ISAVE;
  Save_State() = default;
  explicit Save_State(int n) {
    desc = detail::make_desc(PONNI_LAYER_SAVE_STATE, n, n, ISAVE);
    label = "Save_State";
  }
  void validate() const {}
};

template <int ISAVE, class real = float, int N = 1>
struct Binop_Add : detail::LayerCore {
  static constexpr bool save = false, binop = true;
  static constexpr int index = ISAVE;
  Binop_Add() = default;
  explicit Binop_Add(int n) {
    desc = detail::make_desc(PONNI_LAYER_BINOP_ADD, n, n, ISAVE);
    label = "Binop_Add";
  }
  void validate(int saved_n) const {
    if (saved_n != desc.n_in) abort("ERROR: Saved layer num inputs != this layer's num inputs");
  }
};

template <int ISAVE, class real = float, int N1 = 1, int N2 = 1>
struct Binop_Concatenate : detail::LayerCore {
  static constexpr bool save = false, binop = true;
  static constexpr int index = ISAVE;
  Binop_Concatenate() = default;
  Binop_Concatenate(int num_inputs, int num_outputs, bool after = true) {
    desc = detail::make_desc(PONNI_LAYER_BINOP_CONCATENATE, num_inputs, num_outputs, ISAVE, 0,
                             after ? PONNI_FLAG_CONCAT_AFTER : 0);
    label = "Binop_Concatenate";
  }
  void validate(int saved_n) const {
    if (desc.n_out != saved_n + desc.n_in)
      abort("ERROR: this layer's num outputs != this layer's num inputs + saved layer's num inputs");
  }
};

// out = in + (bias + W^T saved), W [NSAVE, NIN] (ponni_Binop_Projection_Add.h).
template <int ISAVE, class real = float, int NIN = 1, int NSAVE = 1>
struct Binop_Projection_Add : detail::LayerCore {
  static constexpr bool save = false, binop = true;
  static constexpr int index = ISAVE;
  Binop_Projection_Add() = default;
  template <class INIT = Initializer_Random_Uniform<real>>
  Binop_Projection_Add(int num_inputs, int num_saved_inputs, bool trainable_ = true, INIT init = INIT()) {
    std::vector<double> w(static_cast<std::size_t>(num_saved_inputs) * num_inputs), b(num_inputs);
    init.fill(w, num_saved_inputs, num_inputs);
    init.fill(b, num_inputs, num_inputs);
    w.insert(w.end(), b.begin(), b.end());
    setup(num_inputs, num_saved_inputs, std::move(w), trainable_);
  }
  template <class M, class V, class = decltype(std::declval<M const&>()(0, 0))>
  Binop_Projection_Add(M const& weights, V const& bias, bool trainable_ = true) {
    if (static_cast<std::size_t>(weights.extent(1)) != bias.size())
      abort("ERROR: Binop_Projection_Add incompatible weights/bias shapes");
    std::vector<double> p = detail::flatten(weights), b = detail::flatten1(bias);
    p.insert(p.end(), b.begin(), b.end());
    setup(static_cast<int>(weights.extent(1)), static_cast<int>(weights.extent(0)), std::move(p), trainable_);
  }
  void setup(int n_in, int n_save, std::vector<double> p, bool t) {
    desc = detail::make_desc(PONNI_LAYER_BINOP_PROJECTION_ADD, n_in, n_in, ISAVE, n_save);
    params = std::move(p);
    trainable = t;
    label = "Binop_Projection_Add";
  }
  void validate(int saved_n) const {
    if (saved_n != desc.n_aux) abort("ERROR: saved layer size incompatible with projection weights");
  }
};

// ---- the model ---------------------------------------------------------------------------

namespace detail {

template <class L>
inline constexpr bool is_builtin_v = std::is_base_of_v<LayerCore, L>;

// Static flags of a layer type with the reference's defaults.
template <class L, class = void> struct flag_save : std::false_type {};
template <class L> struct flag_save<L, std::void_t<decltype(L::save)>> : std::bool_constant<L::save> {};
template <class L, class = void> struct flag_binop : std::false_type {};
template <class L> struct flag_binop<L, std::void_t<decltype(L::binop)>> : std::bool_constant<L::binop> {};
template <class L, class = void> struct flag_overwrite : std::false_type {};
template <class L>
struct flag_overwrite<L, std::void_t<decltype(L::overwrite_input)>> : std::bool_constant<L::overwrite_input> {};
template <class L, class = void> struct flag_index : std::integral_constant<int, 0> {};
template <class L> struct flag_index<L, std::void_t<decltype(L::index)>> : std::integral_constant<int, L::index> {};

// Device parameters of a layer inside a user-layer chain: the layer's own
// Params for a user layer, nothing for a built-in one (its parameters are in
// the plan's device copy).
struct NoParams {};
template <class L, bool BUILTIN = is_builtin_v<L>>
struct params_of {
  using type = NoParams;
};
template <class L>
struct params_of<L, false> {
  using type = typename L::Params;
};

// The C-ABI descriptor of tuple element I: built-in layers carry theirs; a
// user layer is PONNI_LAYER_EXTERNAL with index I.  A user dense layer never
// runs in place (its outputs read every input feature).
template <int I, class L>
ponni_layer_desc layer_desc(L const& layer) {
  if constexpr (is_builtin_v<L>) {
    return layer.desc;
  } else {
    int flags = 0;
    if (flag_save<L>::value) flags |= PONNI_FLAG_EXT_SAVE;
    if (flag_binop<L>::value) flags |= PONNI_FLAG_EXT_BINOP;
    if (flag_overwrite<L>::value && !is_dense_layer_v<L>) flags |= PONNI_FLAG_EXT_IN_PLACE;
    return make_desc(PONNI_LAYER_EXTERNAL, layer.get_num_inputs(), layer.get_num_outputs(),
                     (flag_save<L>::value || flag_binop<L>::value) ? flag_index<L>::value : 0, 0, flags, double(I));
  }
}

// A per-sample state for user layers' device functions: element (f, b) of
// one of the interpreter's state handles.
template <class real>
struct StateView {
  ponni_hip::View2 v;
  __host__ __device__ real& operator()(int f, int b) const {
    return reinterpret_cast<real*>(v.base)[static_cast<std::int64_t>(f) * v.ld + b];
  }
};

// Batch pass of a chain holding user layers: one sample per thread.
template <class Model, class real>
__global__ __launch_bounds__(256) void user_chain_forward(typename Model::Params p, real const* __restrict__ x,
                                                          std::int64_t ldx, real* __restrict__ y, std::int64_t ldy,
                                                          std::int64_t batch) {
  std::int64_t const b = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b < batch) Model::run_sample(p, x + b, ldx, y + b, ldy);
}

}  // namespace detail

// A model bound to an execution space (HIP: the GPU; Host: host threads);
// Inference<real, Layers...> is the HIP form.
template <class real, class Exec, class... Layers>
class BasicInference {
  static_assert(sizeof...(Layers) > 0, "a model needs at least one layer");
  static_assert(is_execution_space_v<Exec>, "create_inference_model requires an execution space (HIP or Host)");

 public:
  using real_type = real;
  using execution_space = Exec;
  using memory_space = typename Exec::memory_space;
  static constexpr bool runs_on_host = std::is_same_v<memory_space, HostSpace>;
  static_assert(!runs_on_host || std::is_same_v<real, float> || std::is_same_v<real, double>,
                "host execution-space models run in F32 or F64");
  using TUPLE = std::tuple<Layers...>;
  static constexpr int num_layers = static_cast<int>(sizeof...(Layers));
  // A chain holding user layers (the plugin contract) runs one sample per
  // thread through the plan's GENERIC op list, with the user layers' device
  // functions called at their place in it.
  static constexpr bool has_user_layers = !(detail::is_builtin_v<Layers> && ...);
  static_assert(!has_user_layers || std::is_same_v<real, float> || std::is_same_v<real, double>,
                "chains with user layers run in F32 or F64");

  explicit BasicInference(TUPLE const& layers, Exec const& exec = Exec(), int path = PONNI_PATH_AUTO)
      : layers_(layers), exec_(exec) {
    std::vector<ponni_layer_desc> descs;
    collect_descs(descs, std::make_index_sequence<num_layers>{});
    ponni_plan p = nullptr;
    check(ponni_plan_create(descs.data(), num_layers, dtype_of<real>(), path, &p), "create_inference_model");
    plan_ = std::shared_ptr<ponni_plan_s>(p, [](ponni_plan q) { ponni_plan_destroy(q); });
    pushed_.assign(num_layers, ~std::uint64_t(0));
    sync();
  }

  // ---- structure ------------------------------------------------------------------------
  int get_num_inputs() const { return std::get<0>(layers_).get_num_inputs(); }
  int get_num_outputs() const { return std::get<num_layers - 1>(layers_).get_num_outputs(); }
  template <int I>
  auto& get_layer() { return std::get<I>(layers_); }
  template <int I>
  auto const& get_layer() const { return std::get<I>(layers_); }
  hipStream_t stream() const {
    if constexpr (runs_on_host) return nullptr;
    else return exec_.stream;
  }
  Exec const& execution_space_instance() const { return exec_; }
  ponni_plan plan() const { return plan_.get(); }

  ponni_plan_info info() const {
    ponni_plan_info inf{};
    check(ponni_plan_get_info(plan_.get(), &inf), "ponni_plan_get_info");
    return inf;
  }
  // Scratch planning queries of ponni_Inference.h:92-122, :204-223.
  // Dense layers (built-in or user) each start one fused block (ponni_Inference.h:66-85).
  static constexpr int get_num_fused_dense_blocks() { return (int(is_dense_layer_v<Layers>) + ...); }
  int get_num_saved_states() const { return info().num_saved_states; }
  template <int REQUESTED_BUFFER>
  int get_planned_temporary_size() const {
    return REQUESTED_BUFFER == 0 ? info().tmp1_features : info().tmp2_features;
  }

  // Each layer's own validate() plus the chain check (ponni_Inference.h:719-737);
  // the plan already rejected an invalid chain, so this re-checks the layers.
  void validate() const {
    int saved[8] = {};
    std::apply(
        [&](auto const&... l) {
          auto one = [&](auto const& layer) {
            using L = std::decay_t<decltype(layer)>;
            if constexpr (has_save<L>()) {
              if constexpr (L::save) saved[L::index] = layer.get_num_inputs();
            }
            if constexpr (has_binop<L>()) {
              if constexpr (L::binop) layer.validate(saved[L::index]);
              else layer.validate();
            } else {
              layer.validate();
            }
          };
          (one(l), ...);
        },
        layers_);
  }

  void print() const {
    std::cout << "Inference model has " << num_layers << " layers -- with " << get_num_trainable_parameters()
              << " total trainable parameters.\n";
    int i = 0;
    std::apply(
        [&](auto const&... l) {
          ((std::cout << "  " << std::setw(3) << std::right << ++i << ": " << std::setw(15) << std::left
                      << l.get_label() << " with " << l.get_num_inputs() << " inputs, " << l.get_num_outputs()
                      << " outputs, and " << l.get_num_trainable_parameters() << " trainable parameters\n"),
           ...);
        },
        layers_);
  }

  // ---- internal state -------------------------------------------------------------------
  void reallocate_internal_state(int batch_size) {
    if (batch_size < 0) abort("Inference internal-state batch size must be nonnegative");
    check(ponni_plan_reallocate_internal_state(plan_.get(), batch_size), "reallocate_internal_state");
  }
  int internal_state_capacity() const { return static_cast<int>(info().internal_state_capacity); }

  // ---- parameters -----------------------------------------------------------------------
  // Built-in layers' parameters (a user layer keeps its own `params`).
  int get_num_trainable_parameters() const {
    int n = 0;
    std::apply(
        [&](auto const&... l) {
          auto one = [&](auto const& layer) {
            if constexpr (detail::is_builtin_v<std::decay_t<decltype(layer)>>) n += layer.get_num_trainable_parameters();
          };
          (one(l), ...);
        },
        layers_);
    return n;
  }
  // Flattened in tuple order (ponni_Inference.h:688-716).
  std::vector<real> get_trainable_parameters() const {
    std::vector<real> out;
    std::apply(
        [&](auto const&... l) {
          auto one = [&](auto const& layer) {
            if constexpr (detail::is_builtin_v<std::decay_t<decltype(layer)>>)
            for (double v : layer.get_trainable_parameters()) {
              if constexpr (std::is_same_v<real, double>) out.push_back(v);
              else out.push_back(static_cast<real>(static_cast<float>(v)));
            }
          };
          (one(l), ...);
        },
        layers_);
    return out;
  }
  template <class Vec>
  void set_trainable_parameters(Vec const& in) {
    std::size_t off = 0;
    std::apply(
        [&](auto&... l) {
          auto one = [&](auto& layer) {
            if constexpr (!detail::is_builtin_v<std::decay_t<decltype(layer)>>) return;
            else {
            std::size_t const n = static_cast<std::size_t>(layer.get_num_trainable_parameters());
            if (n == 0) return;
            if (in.size() < off + n) abort(std::string("ERROR: ") + layer.get_label() + " trainable input too small");
            std::vector<double> part(n);
            for (std::size_t i = 0; i < n; i++) {
              if constexpr (std::is_same_v<real, double>) part[i] = static_cast<double>(in[off + i]);
              else part[i] = static_cast<double>(static_cast<float>(in[off + i]));
            }
            layer.set_trainable_parameters(part);
            off += n;
            }
          };
          (one(l), ...);
        },
        layers_);
    sync();
  }

  // ---- in-kernel inference (ponni_Inference.h:394-408, :592-665) -----------------------
  // `params` describes the model for application kernels; copy it into the
  // kernel (`auto const p = model.params;`) and call
  // Model::forward_batch_parallel_in_kernel(in, out, p, ibatch) per sample.
  // It is refreshed whenever parameters are pushed (sync()).
  struct UserChainParams {
    ponni_device_model model;
    std::tuple<typename detail::params_of<Layers>::type...> layers;
  };
  using Params = std::conditional_t<has_user_layers, UserChainParams, ponni_device_model>;
  Params params{};

  // Calls user layer `index` of the chain on one sample (the GENERIC
  // interpreter's OP_EXTERNAL callback).
  struct UserLayers {
    Params const* p;
    template <int I>
    __host__ __device__ void call(ponni_hip::View2 const& in, ponni_hip::View2 const& out, ponni_hip::View2 const& sv,
                         int n_out, int b) const {
      using L = std::tuple_element_t<I, TUPLE>;
      if constexpr (!detail::is_builtin_v<L>) {
        auto const& lp = std::get<I>(p->layers);
        detail::StateView<real> const iv{in}, ov{out}, svv{sv};
        if constexpr (is_dense_layer_v<L>) {
          for (int f = 0; f < n_out; f++) ov(f, b) = L::compute_output(iv, f, b, lp);
        } else if constexpr (is_pointwise_layer_v<L>) {
          for (int f = 0; f < n_out; f++) ov(f, b) = apply_fused_layer<L, real>(iv(f, b), f, lp);
        } else if constexpr (detail::flag_binop<L>::value) {
          L::compute_all_outputs(iv, svv, ov, b, lp);
        } else {
          L::compute_all_outputs(iv, ov, b, lp);
        }
      }
    }
    template <std::size_t... I>
    __host__ __device__ void dispatch(int index, ponni_hip::View2 const& in, ponni_hip::View2 const& out,
                             ponni_hip::View2 const& sv, int n_out, int b, std::index_sequence<I...>) const {
      ((index == static_cast<int>(I) ? (call<static_cast<int>(I)>(in, out, sv, n_out, b), 0) : 0), ...);
    }
    __host__ __device__ void operator()(int index, int, ponni_hip::View2 const& in, ponni_hip::View2 const& out,
                               ponni_hip::View2 const& sv, int, int n_out, std::int64_t b) const {
      dispatch(index, in, out, sv, n_out, static_cast<int>(b), std::make_index_sequence<num_layers>{});
    }
  };

  // One sample: column pointers with row strides (thread-private states).
  template <int MAXW = kInKernelMaxWidth, int MAXSAVED = kInKernelMaxSaved>
  __host__ __device__ static void run_sample(Params const& p, real const* in, std::int64_t in_ld, real* out,
                                    std::int64_t out_ld) {
    static_assert(std::is_same_v<real, float> || std::is_same_v<real, double>,
                  "in-kernel inference runs F32 and F64 models");
    if constexpr (has_user_layers) forward_one<real, MAXW, MAXSAVED>(p.model, in, in_ld, out, out_ld, UserLayers{&p});
    else forward_one<real, MAXW, MAXSAVED>(p, in, in_ld, out, out_ld);
  }

  // Sample `ibatch` of LayoutRight [features, batch] views (device memory).
  template <class InputView, class OutputView, int MAXW = kInKernelMaxWidth, int MAXSAVED = kInKernelMaxSaved>
  __host__ __device__ static void forward_batch_parallel_in_kernel(InputView const& input, OutputView const& output,
                                                          Params const& p, int ibatch) {
    run_sample<MAXW, MAXSAVED>(p, input.data() + ibatch, input.stride(0), output.data() + ibatch, output.stride(0));
  }
  // One sample held in per-thread arrays.
  template <int NI, int NO, int MAXW = kInKernelMaxWidth, int MAXSAVED = kInKernelMaxSaved>
  __host__ __device__ static void forward_batch_parallel_in_kernel(SArray<real, NI> const& input, SArray<real, NO>& output,
                                                          Params const& p) {
    run_sample<MAXW, MAXSAVED>(p, input.data(), 1, output.data(), 1);
  }

  // Push parameters of layers changed since the last push (set_trainable_parameters,
  // or get_layer<I>() edits followed by mark_modified()).
  void sync() {
    int i = 0;
    std::apply(
        [&](auto const&... l) {
          auto one = [&](auto const& layer) {
            if constexpr (!detail::is_builtin_v<std::decay_t<decltype(layer)>>) {
              i++;
              return;
            } else {
            if (pushed_[i] != layer.version && !layer.params.empty()) {
              std::vector<float> f;
              void const* src = layer.params.data();
              if constexpr (!std::is_same_v<real, double>) {
                f.assign(layer.params.begin(), layer.params.end());
                src = f.data();
              }
              check(ponni_plan_set_layer_params(plan_.get(), i, src, static_cast<std::int64_t>(layer.params.size())),
                    "ponni_plan_set_layer_params");
            }
            pushed_[i] = layer.version;
            i++;
            }
          };
          (one(l), ...);
        },
        layers_);
    // Host models describe the plan in host memory; device models do so only
    // where a device exists (models are also built on GPU-less hosts).
    int devices = 0;
    if constexpr (runs_on_host) {
      if constexpr (has_user_layers) {
        check(ponni_plan_host_model(plan_.get(), &params.model), "ponni_plan_host_model");
        collect_user_params(std::make_index_sequence<num_layers>{});
      } else {
        check(ponni_plan_host_model(plan_.get(), &params), "ponni_plan_host_model");
      }
    } else if constexpr (std::is_same_v<real, float> || std::is_same_v<real, double>) {
      if (hipGetDeviceCount(&devices) == hipSuccess && devices > 0) {
        if constexpr (has_user_layers) {
          check(ponni_plan_device_model(plan_.get(), &params.model), "ponni_plan_device_model");
          collect_user_params(std::make_index_sequence<num_layers>{});
        } else {
          check(ponni_plan_device_model(plan_.get(), &params), "ponni_plan_device_model");
        }
      }
    }
  }

  // ---- weights files (ponni_Inference.h:270-333) ---------------------------------------------
  std::string weight_schema_fingerprint() const {
    std::vector<char const*> labels;
    std::vector<std::int32_t> nin, nout;
    std::vector<std::int64_t> ntr;
    std::apply(
        [&](auto const&... l) {
          ((labels.push_back(l.get_label()), nin.push_back(l.get_num_inputs()), nout.push_back(l.get_num_outputs()),
            ntr.push_back(l.get_num_trainable_parameters())),
           ...);
        },
        layers_);
    char buf[64];
    check(ponni_template_fingerprint(num_layers, labels.data(), nin.data(), nout.data(), ntr.data(), buf, sizeof(buf)),
          "weight_schema_fingerprint");
    return buf;
  }

  bool save_weights(std::string const& path, std::string* error = nullptr) const {
    int const n = get_num_trainable_parameters();
    if (n == 0) {
      if (error) *error = "cannot save weights from a model with no trainable parameters";
      return false;
    }
    std::vector<real> p = get_trainable_parameters();
    int st;
    if constexpr (std::is_same_v<real, double>) {
      st = ponni_file_write_parameters(path.c_str(), weight_schema_fingerprint().c_str(), p.data(), n, 8, "template");
    } else {
      std::vector<float> f(p.begin(), p.end());
      st = ponni_file_write_parameters(path.c_str(), weight_schema_fingerprint().c_str(), f.data(), n, 4, "template");
    }
    if (st != PONNI_OK && error) *error = ponni_last_error();
    return st == PONNI_OK;
  }

  bool load_weights(std::string const& path, std::string* error = nullptr) {
    int const n = get_num_trainable_parameters();
    if (n == 0) {
      if (error) *error = "cannot load weights into a model with no trainable parameters";
      return false;
    }
    int st;
    if constexpr (std::is_same_v<real, double>) {
      std::vector<double> v(n);
      st = ponni_file_read_parameters(path.c_str(), weight_schema_fingerprint().c_str(), v.data(), n, 8);
      if (st == PONNI_OK) set_trainable_parameters(v);
    } else {
      std::vector<float> v(n);
      st = ponni_file_read_parameters(path.c_str(), weight_schema_fingerprint().c_str(), v.data(), n, 4);
      if (st == PONNI_OK) set_trainable_parameters(v);
    }
    if (st != PONNI_OK && error) *error = ponni_last_error();
    return st == PONNI_OK;
  }

  // ---- inference --------------------------------------------------------------------------
  // Allocates and zero-fills the output, then runs (ponni_Inference.h:338-346).
  template <class InputView>
  View<real, memory_space> forward_batch_parallel(InputView const& input) {
    require_layout_right_views<InputView>();
    std::int64_t const batch = static_cast<std::int64_t>(input.extent(1));
    if (batch == 0) abort("Inference requires a nonzero batch size");
    View<real, memory_space> output("output", get_num_outputs(), batch, true);
    forward_batch_parallel(input, output);
    return output;
  }

  // Into caller-provided storage (ponni_Inference.h:352-389): asynchronous on
  // the model's stream for HIP models, synchronous for host models.
  template <class InputView, class OutputView>
  void forward_batch_parallel(InputView const& input, OutputView const& output) {
    require_layout_right_views<InputView, OutputView>();
    static_assert(std::is_same_v<typename view_memory_space<InputView>::type, memory_space> &&
                      std::is_same_v<typename view_memory_space<OutputView>::type, memory_space>,
                  "Inference Views must live in the model's memory space");
    static_assert(!std::is_const_v<std::remove_pointer_t<decltype(output.data())>>,
                  "Inference output View must be writable");
    std::int64_t const batch = static_cast<std::int64_t>(input.extent(1));
    if (batch == 0) abort("Inference requires a nonzero batch size");
    if (static_cast<int>(input.extent(0)) != get_num_inputs())
      abort("Error: Provided # inputs differs from model's # inputs");
    if (static_cast<int>(output.extent(0)) != get_num_outputs() || output.extent(1) != input.extent(1))
      abort("Error: Provided output dimensions do not match the model and input batch");
    sync();
    if constexpr (runs_on_host) {
      if constexpr (has_user_layers) {
        if (!fits_in_kernel(params.model)) abort("Error: a chain with user layers is limited to 256-feature states");
        for (std::int64_t b = 0; b < batch; b++)
          run_sample(params, input.data() + b, static_cast<std::int64_t>(input.stride(0)), output.data() + b,
                     static_cast<std::int64_t>(output.stride(0)));
      } else {
        check(ponni_forward_host(plan_.get(), input.data(), static_cast<std::int64_t>(input.stride(0)), output.data(),
                                 static_cast<std::int64_t>(output.stride(0)), batch, exec_.threads),
              "forward_batch_parallel");
      }
    } else if constexpr (has_user_layers) {
      if (!fits_in_kernel(params.model)) abort("Error: a chain with user layers is limited to 256-feature states");
      unsigned const blocks = static_cast<unsigned>((batch + 255) / 256);
      hipLaunchKernelGGL((detail::user_chain_forward<BasicInference, real>), dim3(blocks), dim3(256), 0, stream(), params,
                         input.data(), static_cast<std::int64_t>(input.stride(0)), output.data(),
                         static_cast<std::int64_t>(output.stride(0)), batch);
      hipError_t const e = hipGetLastError();
      if (e != hipSuccess) abort(std::string("forward_batch_parallel: ") + hipGetErrorString(e));
    } else {
      check(ponni_forward(plan_.get(), input.data(), static_cast<std::int64_t>(input.stride(0)), output.data(),
                          static_cast<std::int64_t>(output.stride(0)), batch, stream()),
            "forward_batch_parallel");
    }
  }

 private:
  template <class L>
  static constexpr bool has_save() {
    return has_member_save<L>(0);
  }
  template <class L>
  static constexpr bool has_binop() {
    return has_member_binop<L>(0);
  }
  template <class L>
  static constexpr auto has_member_save(int) -> decltype(L::save, true) {
    return true;
  }
  template <class L>
  static constexpr bool has_member_save(long) {
    return false;
  }
  template <class L>
  static constexpr auto has_member_binop(int) -> decltype(L::binop, true) {
    return true;
  }
  template <class L>
  static constexpr bool has_member_binop(long) {
    return false;
  }

  template <std::size_t... I>
  void collect_descs(std::vector<ponni_layer_desc>& descs, std::index_sequence<I...>) const {
    (descs.push_back(detail::layer_desc<static_cast<int>(I)>(std::get<I>(layers_))), ...);
  }
  template <std::size_t... I>
  void collect_user_params(std::index_sequence<I...>) {
    auto one = [&](auto idx) {
      constexpr std::size_t k = decltype(idx)::value;
      if constexpr (!detail::is_builtin_v<std::tuple_element_t<k, TUPLE>>)
        std::get<k>(params.layers) = std::get<k>(layers_).params;
    };
    (one(std::integral_constant<std::size_t, I>{}), ...);
  }

  TUPLE layers_;
  Exec exec_;
  std::shared_ptr<ponni_plan_s> plan_;
  std::vector<std::uint64_t> pushed_;
};

// ---- View copies and .ponni tensors (src/utils/ponni_view_ops.h:12-48,
// src/utils/ponni_safetensors.h:409-444) ------------------------------------------------

// A copy of `v` in memory space Space (LayoutRight, contiguous rows).
template <class Space, class T, class S>
View<std::remove_const_t<T>, Space> create_memory_space_copy(View<T, S> const& v, Space = Space()) {
  View<std::remove_const_t<T>, Space> out(v.label(), v.extent(0), v.extent(1), false);
  out.copy_from_host(v.copy_to_host());
  return out;
}
template <class T, class S>
View<std::remove_const_t<T>, HostSpace> create_host_copy(View<T, S> const& v) {
  return create_memory_space_copy<HostSpace>(v);
}
template <class T, class S>
View<std::remove_const_t<T>, HIPSpace> create_device_copy(View<T, S> const& v) {
  return create_memory_space_copy<HIPSpace>(v);
}
// The elements of a contiguous view as one row, sharing its memory.
template <class T, class S>
View<T, S> flatten(View<T, S> const& v) {
  return v.reshape(1, v.size());
}

// Tensor `name` of a .ponni file as a float View in Space: rank 2 [rows, cols];
// rank 1 [1, n] (this View type is rank 2).  F32 or F64 payloads.
template <int N, class Space = HIPSpace>
View<float, Space> load_ponni_tensor(PonniFile const& file, std::string const& name) {
  static_assert(N == 1 || N == 2, "load_ponni_tensor supports ranks one and two");
  auto const* t = file.find(name);
  if (t == nullptr) throw std::runtime_error("PONNI file is missing tensor " + name);
  if (t->shape.size() != static_cast<std::size_t>(N)) throw std::runtime_error("PONNI tensor rank mismatch for " + name);
  if (t->dtype != "F32" && t->dtype != "F64") throw std::runtime_error("PONNI tensor must use F32 or F64: " + name);
  std::int64_t const rows = N == 1 ? 1 : static_cast<std::int64_t>(t->shape[0]);
  std::int64_t const cols = static_cast<std::int64_t>(t->shape[N - 1]);
  std::vector<float> h(static_cast<std::size_t>(rows * cols));
  unsigned char const* data = file.tensor_data(*t);
  for (std::size_t i = 0; i < h.size(); i++) {
    if (t->dtype == "F32") {
      float v;
      std::memcpy(&v, data + 4 * i, 4);
      h[i] = v;
    } else {
      double v;
      std::memcpy(&v, data + 8 * i, 8);
      h[i] = static_cast<float>(v);
    }
  }
  View<float, Space> out(name, rows, cols, false);
  out.copy_from_host(h);
  return out;
}
template <int N, class Space = HIPSpace>
View<float, Space> load_ponni_tensor(std::string const& path, std::string const& name) {
  PonniFile file;
  std::string error;
  if (!file.load(path, &error)) throw std::runtime_error(error);
  return load_ponni_tensor<N, Space>(file, name);
}

// ---- factories (ponni_create_model.h:40-98) ------------------------------------------------

template <class real, class... Layers>
using Inference = BasicInference<real, HIP, Layers...>;

namespace detail {
template <class real, class Exec, class Mem, class... Layers>
inline auto create_model(Exec const& exec, Mem const&, Layers const&... layers) {
  static_assert(is_execution_space_v<Exec>, "create_inference_model requires an execution space (HIP or Host)");
  static_assert(is_memory_space_v<Mem>, "create_inference_model requires a memory space (HIPSpace or HostSpace)");
  static_assert(std::is_same_v<typename Exec::memory_space, Mem>,
                "create_inference_model execution space cannot access its memory space");
  return BasicInference<real, Exec, Layers...>(std::make_tuple(layers...), exec);
}
}  // namespace detail

// Layers are copied into the model (parameters live in the plan's buffers),
// as the reference deep-copies them when the memory space differs.
template <class First, class... Rest,
          std::enable_if_t<!is_execution_space_v<First> && !std::is_same_v<std::decay_t<First>, hipStream_t>, int> = 0>
inline auto create_inference_model(First const& first, Rest const&... rest) {
  return Inference<float, First, Rest...>(std::make_tuple(first, rest...));
}
// The execution-space-instance overloads (ponni_create_model.h:52-78).
template <class Exec, class... Layers, std::enable_if_t<is_execution_space_v<Exec>, int> = 0>
inline auto create_inference_model(Exec const& exec, Layers const&... layers) {
  return detail::create_model<float>(exec, typename Exec::memory_space(), layers...);
}
template <class Exec, class Mem, class... Layers,
          std::enable_if_t<is_execution_space_v<Exec> && is_memory_space_v<Mem>, int> = 0>
inline auto create_inference_model(Exec const& exec, Mem const& mem, Layers const&... layers) {
  return detail::create_model<float>(exec, mem, layers...);
}
// A HIP stream is the HIP execution-space instance.
template <class... Layers>
inline auto create_inference_model(hipStream_t stream, Layers const&... layers) {
  return Inference<float, Layers...>(std::make_tuple(layers...), HIP(stream));
}
template <class... Layers>
inline auto create_inference_model_single_precision(Layers const&... layers) {
  return Inference<float, Layers...>(std::make_tuple(layers...));
}
template <class... Layers>
inline auto create_inference_model_double_precision(Layers const&... layers) {
  return Inference<double, Layers...>(std::make_tuple(layers...));
}
template <class... Layers>
inline auto create_inference_model_half_precision(Layers const&... layers) {
  return Inference<half_t, Layers...>(std::make_tuple(layers...));
}
template <class... Layers>
inline auto create_inference_model_bhalf_precision(Layers const&... layers) {
  return Inference<bhalf_t, Layers...>(std::make_tuple(layers...));
}

}  // namespace ponni
