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
//   - initializers               src/initializers/ponni_initializer.h (all fifteen)
//   - .ponni files               src/utils/ponni_safetensors.h via ponni/ponni_file.h,
//                                load_ponni_tensor and the View copies of
//                                src/utils/ponni_view_ops.h
//
// What changes underneath: the per-sample Kokkos RangePolicy executor is
// replaced by one call of ponni_forward(), which runs a gfx950 kernel chosen
// (and, for wide models, generated) for the whole layer chain.  Models bound
// to the host execution space (create_inference_model(Host(), HostSpace(),
// ...)) run on host threads through ponni_forward_host instead, on host
// Views.  Layers hold their parameters in Views of their memory space
// (`params.weights`, ...); create_inference_model rebinds every layer to the
// model's memory space (a copy only when the spaces differ) and the model
// shares the layers' Views with its plan, which re-reads them at every
// forward pass into its kernel layout (ponni_plan_share_layer_params), so a
// write through a layer's View reaches the next pass, as in the reference.
// A View here is ponni::View<T**, Space> / View<T*, Space> (View<T, Space>
// is rank 2 too), or any type with data(), extent(), stride(), a
// memory_space and a LayoutRight array_layout, such as a Kokkos::View with
// Kokkos::LayoutRight: a foreign view of the layer's element type and memory
// space is shared, any other one copied through the runtime (device memory
// is never read on the host).
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
#include "ponni/two_half.h"
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

// Trivially copyable handle of a rank-2 View for device code (kernel
// arguments, lambda captures): the same accessors, no ownership.
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
// device pointer is what forward_batch_parallel has always taken).  Kokkos
// memory spaces map by accessibility: host-accessible ones are HostSpace.
template <class V, class = void> struct view_memory_space { using type = HIPSpace; };
template <class V> struct view_memory_space<V, std::void_t<typename V::memory_space>> {
#ifdef KOKKOS_VERSION
  using type = std::conditional_t<
      std::is_same_v<typename V::memory_space, HostSpace> ||
          Kokkos::SpaceAccessibility<Kokkos::DefaultHostExecutionSpace, typename V::memory_space>::accessible,
      HostSpace, HIPSpace>;
#else
  using type = std::conditional_t<std::is_same_v<typename V::memory_space, HostSpace>, HostSpace, HIPSpace>;
#endif
};

namespace detail {
// View<T, S> and View<T**, S> are rank 2, View<T*, S> rank 1 (the Kokkos
// data-type spelling; the plain element type is kept for rank 2).
template <class D> struct view_data { using value_type = D; static constexpr int rank = 2; };
template <class T> struct view_data<T*> { using value_type = T; static constexpr int rank = 1; };
template <class T> struct view_data<T**> { using value_type = T; static constexpr int rank = 2; };
[[noreturn]] inline void view_abort(std::string const& message) {
  std::fprintf(stderr, "%s\n", message.c_str());
  std::fflush(stderr);
  std::abort();
}
inline void view_check(hipError_t e, char const* what) {
  if (e != hipSuccess) view_abort(std::string(what) + ": " + hipGetErrorString(e));
}
}  // namespace detail

// A LayoutRight array in device memory (HIPSpace, the default) or host memory
// (HostSpace): rank 2 [rows, cols] with element (r, c) at
// data()[r * stride(0) + c], or rank 1 [n], contiguous.  Copies share the
// allocation (as Kokkos::View does).
template <class D, class Space = HIPSpace>
class View {
  static_assert(is_memory_space_v<Space>, "ponni::View memory space must be HIPSpace or HostSpace");
  static constexpr bool on_host = std::is_same_v<Space, HostSpace>;
  template <class, class> friend class View;

 public:
  using value_type = typename detail::view_data<D>::value_type;
  using T = value_type;
  using non_const_value_type = std::remove_const_t<T>;
  using array_layout = LayoutRight;
  using memory_space = Space;
  static constexpr int rank = detail::view_data<D>::rank;

  View() = default;
  // rank 2: [rows, cols]; rank 1: View(label, n).  Device arrays start at zero
  // unless `zero` is false; host arrays always do.
  View(std::string label, std::int64_t rows, std::int64_t cols, bool zero = true) : label_(std::move(label)) {
    static_assert(rank == 2, "a rank-1 View takes one extent");
    allocate(rows, cols, zero);
  }
  View(std::string label, std::int64_t n) : label_(std::move(label)) {
    static_assert(rank == 1, "a rank-2 View takes two extents");
    allocate(1, n, true);
  }
  // The same array under another spelling of the same rank (View<T> <-> View<T**>).
  template <class D2, class = std::enable_if_t<!std::is_same_v<D2, D> && detail::view_data<D2>::rank == rank &&
                                               std::is_same_v<typename detail::view_data<D2>::value_type, T>>>
  View(View<D2, Space> const& o)
      : label_(o.label_), owner_(o.owner_), data_(o.data_), rows_(o.rows_), cols_(o.cols_), ld_(o.ld_) {}

  // Caller-owned memory of this space (no ownership; `keep` holds whatever
  // keeps it alive, e.g. the foreign view it came from).
  static View wrap(T* data, std::int64_t rows, std::int64_t cols, std::int64_t ld,
                   std::shared_ptr<void> keep = nullptr) {
    View v;
    v.data_ = data;
    v.rows_ = rows;
    v.cols_ = cols;
    v.ld_ = ld;
    v.owner_ = std::move(keep);
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
    static_assert(rank == 2, "reshape makes a rank-2 View");
    if (rows * cols != size() || !contiguous()) detail::view_abort("ponni::View::reshape needs a contiguous view of the same size");
    View v = *this;
    v.rows_ = rows;
    v.cols_ = cols;
    v.ld_ = cols;
    return v;
  }

  __host__ __device__ T* data() const { return data_; }
  __host__ __device__ std::int64_t extent(int d) const {
    if constexpr (rank == 1) return d == 0 ? cols_ : 1;
    else return d == 0 ? rows_ : cols_;
  }
  __host__ __device__ std::int64_t stride(int d) const {
    if constexpr (rank == 1) return 1;
    else return d == 0 ? ld_ : 1;
  }
  __host__ __device__ T& operator()(std::int64_t r, std::int64_t c) const { return data_[r * ld_ + c]; }
  __host__ __device__ T& operator()(std::int64_t i) const {
    static_assert(rank == 1, "a rank-2 View takes two indices");
    return data_[i];
  }
  DeviceView<T> device() const { return DeviceView<T>{data_, rows_, cols_, ld_}; }
  std::int64_t size() const { return rows_ * cols_; }
  std::int64_t rows() const { return rows_; }  // rank 1: 1
  std::int64_t cols() const { return cols_; }  // rank 1: n
  std::int64_t ld() const { return ld_; }
  bool contiguous() const { return rows_ <= 1 || ld_ == cols_; }
  bool is_allocated() const { return data_ != nullptr; }
  std::string const& label() const { return label_; }
  std::shared_ptr<void> const& owner() const { return owner_; }

  // Copies from / to a row-major host array of size() elements.
  void copy_from_host(std::vector<non_const_value_type> const& h) const {
    if (static_cast<std::int64_t>(h.size()) != size()) detail::view_abort("ponni::View::copy_from_host size mismatch");
    if (size() == 0) return;
    if constexpr (on_host) {
      for (std::int64_t r = 0; r < rows_; r++)
        std::memcpy(const_cast<non_const_value_type*>(data_) + r * ld_, h.data() + r * cols_, sizeof(T) * cols_);
    } else {
      detail::view_check(hipMemcpy2D(const_cast<non_const_value_type*>(data_), sizeof(T) * ld_, h.data(),
                                     sizeof(T) * cols_, sizeof(T) * cols_, rows_, hipMemcpyHostToDevice),
                         "hipMemcpy2D");
    }
  }
  std::vector<non_const_value_type> copy_to_host() const {
    std::vector<non_const_value_type> h(static_cast<std::size_t>(size()));
    if (size() == 0) return h;
    if constexpr (on_host) {
      for (std::int64_t r = 0; r < rows_; r++) std::memcpy(h.data() + r * cols_, data_ + r * ld_, sizeof(T) * cols_);
    } else {
      detail::view_check(hipMemcpy2D(h.data(), sizeof(T) * cols_, data_, sizeof(T) * ld_, sizeof(T) * cols_, rows_,
                                     hipMemcpyDeviceToHost),
                         "hipMemcpy2D");
    }
    return h;
  }

 private:
  void allocate(std::int64_t rows, std::int64_t cols, bool zero) {
    if (rows < 0 || cols < 0) detail::view_abort("ponni::View extents must be nonnegative");
    rows_ = rows;
    cols_ = cols;
    ld_ = cols;
    if (rows * cols == 0) return;
    std::size_t const bytes = sizeof(T) * static_cast<std::size_t>(rows * cols);
    void* p = nullptr;
    if constexpr (on_host) {
      p = std::calloc(static_cast<std::size_t>(rows * cols), sizeof(T));
      if (p == nullptr) detail::view_abort("ponni::View host allocation failed");
      owner_ = std::shared_ptr<void>(p, [](void* q) { std::free(q); });
    } else {
      detail::view_check(hipMalloc(&p, bytes), "hipMalloc");
      if (zero) detail::view_check(hipMemset(p, 0, bytes), "hipMemset");
      owner_ = std::shared_ptr<void>(p, [](void* q) { (void)hipFree(q); });
    }
    data_ = static_cast<T*>(p);
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

// ---- View operations (src/utils/ponni_view_ops.h:12-48) ----------------------------------

// A copy of `v` in memory space Space (LayoutRight, contiguous rows).
template <class Space, class D, class S>
View<std::remove_const_t<D>, Space> create_memory_space_copy(View<D, S> const& v, Space = Space()) {
  using R = View<std::remove_const_t<D>, Space>;
  R out;
  if constexpr (R::rank == 1) out = R(v.label(), v.extent(0));
  else out = R(v.label(), v.extent(0), v.extent(1), false);
  out.copy_from_host(v.copy_to_host());
  return out;
}
template <class D, class S>
View<std::remove_const_t<D>, HostSpace> create_host_copy(View<D, S> const& v) {
  return create_memory_space_copy<HostSpace>(v);
}
template <class D, class S>
View<std::remove_const_t<D>, HIPSpace> create_device_copy(View<D, S> const& v) {
  return create_memory_space_copy<HIPSpace>(v);
}
// The elements of a contiguous rank-2 View as a rank-1 View, sharing its memory.
template <class D, class S>
View<typename View<D, S>::value_type*, S> flatten(View<D, S> const& v) {
  if (!v.contiguous()) detail::view_abort("ponni::flatten needs a contiguous View");
  return View<typename View<D, S>::value_type*, S>::wrap(v.data(), 1, v.size(), v.size(), v.owner());
}
// Every element of `dst` set to `value` (Kokkos::deep_copy(view, scalar)).
template <class D, class S>
void deep_copy(View<D, S> const& dst, typename View<D, S>::value_type const& value) {
  dst.copy_from_host(std::vector<typename View<D, S>::non_const_value_type>(static_cast<std::size_t>(dst.size()), value));
}
// Element-wise copy between Views of the same size, in any memory spaces
// (Kokkos::deep_copy(dst, src); sizes must match).
template <class D1, class S1, class D2, class S2>
void deep_copy(View<D1, S1> const& dst, View<D2, S2> const& src) {
  if (dst.size() != src.size()) detail::view_abort("ponni::deep_copy: Views differ in size");
  auto h = src.copy_to_host();
  std::vector<typename View<D1, S1>::non_const_value_type> out(h.begin(), h.end());
  dst.copy_from_host(out);
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
// A seed of 0 draws a fresh one from the clock (ponni_initializer.h:20-22).
inline std::uint64_t effective_seed(std::uint64_t seed) {
  return seed == 0 ? static_cast<std::uint64_t>(std::time(nullptr)) : seed;
}
// Draw k of element i's own stream, uniform on [0, 1) (53 random bits); each
// element has its own stream so a fill does not depend on thread scheduling.
inline double unit(std::uint64_t seed, std::uint64_t i, std::uint64_t k = 0) {
  return static_cast<double>(splitmix64(seed ^ splitmix64(splitmix64(i + 1) + k)) >> 11) *
         (1.0 / 9007199254740992.0);
}
// Standard normal draw k of element i (Box-Muller on two uniforms).
inline double normal(std::uint64_t seed, std::uint64_t i, std::uint64_t k = 0) {
  double const u1 = 1.0 - unit(seed, i, 2 * k), u2 = unit(seed, i, 2 * k + 1);
  return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}
inline void require_finite(double v, char const* message) {
  if (!std::isfinite(v)) throw std::invalid_argument(message);
}
// The value as `real` holds it, kept below `ub` when the rounding of a draw
// just under ub would reach it (bounds are half-open, as drand(lb, ub)).
template <class real>
double as_real(double v) {
  if constexpr (std::is_same_v<real, double>) return v;
  else return static_cast<double>(static_cast<float>(static_cast<real>(static_cast<float>(v))));
}
template <class real>
double below(double v, double lb, double ub) {
  if (as_real<real>(v) < ub || !(lb < ub)) return v;
  if constexpr (std::is_same_v<real, double>) return std::nextafter(ub, lb);
  float f = static_cast<float>(ub);
  while (as_real<real>(f) >= ub) f = std::nextafter(f, -INFINITY);
  return f;
}
template <class real>
void fill_uniform(std::vector<double>& a, double lb, double ub, std::uint64_t seed) {
  if (a.empty()) return;
  if (lb == ub) {
    for (double& v : a) v = lb;
    return;
  }
  std::uint64_t const s = effective_seed(seed);
  for (std::size_t i = 0; i < a.size(); i++) a[i] = below<real>(lb + (ub - lb) * unit(s, i), lb, ub);
}
inline void fill_normal(std::vector<double>& a, double mean, double stdev, std::uint64_t seed) {
  if (a.empty()) return;
  std::uint64_t const s = effective_seed(seed);
  for (std::size_t i = 0; i < a.size(); i++) a[i] = stdev == 0.0 ? mean : mean + stdev * normal(s, i);
}
// Normal draws outside mean +- 2 stdev are drawn again (ponni_initializer.h:143-161).
inline void fill_truncated_normal(std::vector<double>& a, double mean, double stdev, std::uint64_t seed) {
  if (a.empty()) return;
  std::uint64_t const s = effective_seed(seed);
  for (std::size_t i = 0; i < a.size(); i++) {
    if (stdev == 0.0) {
      a[i] = mean;
      continue;
    }
    double z = normal(s, i, 0);
    for (std::uint64_t k = 1; std::abs(z) > 2.0; k++) z = normal(s, i, k);
    a[i] = mean + stdev * z;
  }
}
// Gram-Schmidt over the columns of a [m, n] array when m >= n, else over its
// rows, then scaled by `gain` (ponni_initializer.h:313-377).
inline void orthonormalize(std::vector<double>& a, int m, int n, double gain) {
  auto at = [&](int i, int j) -> double& { return a[static_cast<std::size_t>(i) * n + j]; };
  bool const cols = m >= n;
  int const count = cols ? n : m, len = cols ? m : n;
  auto el = [&](int vec, int k) -> double& { return cols ? at(k, vec) : at(vec, k); };
  for (int j = 0; j < count; j++) {
    for (int k = 0; k < j; k++) {
      double dot = 0;
      for (int i = 0; i < len; i++) dot += el(j, i) * el(k, i);
      for (int i = 0; i < len; i++) el(j, i) -= dot * el(k, i);
    }
    double norm = 0;
    for (int i = 0; i < len; i++) norm += el(j, i) * el(j, i);
    norm = std::sqrt(norm) + 1e-20;
    for (int i = 0; i < len; i++) el(j, i) /= norm;
  }
  for (double& v : a) v *= gain;
}
// fan_in / fan_out of a [n_in, n_out] array (a rank-1 one: its length for
// both), ponni_initializer.h:89-107.
template <class V>
void fans(V const& a, double& fan_in, double& fan_out) {
  fan_in = static_cast<double>(a.extent(0));
  fan_out = V::rank >= 2 ? static_cast<double>(a.extent(1)) : fan_in;
}
// Apply a flat fill to any View (values made on the host, then copied in).
template <class V, class F>
void fill_view(V const& a, F&& fill) {
  std::vector<double> v(static_cast<std::size_t>(a.size()));
  fill(v);
  using T = typename V::non_const_value_type;
  std::vector<T> out(v.size());
  for (std::size_t i = 0; i < v.size(); i++) {
    if constexpr (std::is_same_v<T, double>) out[i] = v[i];
    else out[i] = static_cast<T>(static_cast<float>(v[i]));
  }
  a.copy_from_host(out);
}
}  // namespace init_detail

// Initializers of src/initializers/ponni_initializer.h: the same names,
// parameters, validation (std::invalid_argument), fan conventions (a
// [n_in, n_out] array has fan_in = n_in, fan_out = n_out) and degenerate
// cases; fill(view) works on a View in either memory space.  The random
// streams are this library's own (splitmix64, one stream per element; seed 0
// draws from the clock); the reference's Kokkos XorShift streams are not
// reproduced, so fills agree with the reference in distribution only.
template <class real>
struct Initializer_None {
  template <class V> void fill(V const&) const { require_layout_right_views<V>(); }
  void fill(std::vector<double>&, int, int) const {}
};
template <class real>
struct Initializer_Random_Uniform {
  real lb, ub;
  std::uint64_t seed;
  Initializer_Random_Uniform(real lb_ = real(-0.05), real ub_ = real(0.05), std::uint64_t seed_ = 0)
      : lb(lb_), ub(ub_), seed(seed_) {
    init_detail::require_finite(static_cast<double>(lb), "Initializer_Random_Uniform lower bound must be finite");
    init_detail::require_finite(static_cast<double>(ub), "Initializer_Random_Uniform upper bound must be finite");
    if (static_cast<double>(lb) > static_cast<double>(ub))
      throw std::invalid_argument("Initializer_Random_Uniform requires lower bound <= upper bound");
  }
  void fill(std::vector<double>& a, int, int) const {
    init_detail::fill_uniform<real>(a, static_cast<double>(lb), static_cast<double>(ub), seed);
  }
  template <class V> void fill(V const& a) const {
    init_detail::fill_view(a, [&](std::vector<double>& v) { fill(v, 0, 0); });
  }
};
template <class real>
struct Initializer_Constant {
  real value;
  explicit Initializer_Constant(real v = real(0)) : value(v) {}
  void fill(std::vector<double>& a, int, int) const {
    for (double& v : a) v = static_cast<double>(value);
  }
  template <class V> void fill(V const& a) const {
    init_detail::fill_view(a, [&](std::vector<double>& v) { fill(v, 0, 0); });
  }
};
template <class real> struct Initializer_Zeros : Initializer_Constant<real> { Initializer_Zeros() : Initializer_Constant<real>(real(0)) {} };
template <class real> struct Initializer_Ones : Initializer_Constant<real> { Initializer_Ones() : Initializer_Constant<real>(real(1)) {} };
template <class real>
struct Initializer_Random_Normal {
  real mean, stdev;
  std::uint64_t seed;
  Initializer_Random_Normal(real m = real(0), real s = real(1), std::uint64_t sd = 0) : mean(m), stdev(s), seed(sd) {
    init_detail::require_finite(static_cast<double>(mean), "Initializer_Random_Normal mean must be finite");
    init_detail::require_finite(static_cast<double>(stdev), "Initializer_Random_Normal standard deviation must be finite");
    if (static_cast<double>(stdev) < 0)
      throw std::invalid_argument("Initializer_Random_Normal standard deviation must be nonnegative");
  }
  void fill(std::vector<double>& a, int, int) const {
    init_detail::fill_normal(a, static_cast<double>(mean), static_cast<double>(stdev), seed);
  }
  template <class V> void fill(V const& a) const {
    init_detail::fill_view(a, [&](std::vector<double>& v) { fill(v, 0, 0); });
  }
};
template <class real>
struct Initializer_Truncated_Normal {
  real mean, stdev;
  std::uint64_t seed;
  Initializer_Truncated_Normal(real m = real(0), real s = real(1), std::uint64_t sd = 0)
      : mean(m), stdev(s), seed(sd) {
    init_detail::require_finite(static_cast<double>(mean), "Initializer_Truncated_Normal mean must be finite");
    init_detail::require_finite(static_cast<double>(stdev),
                                "Initializer_Truncated_Normal standard deviation must be finite");
    if (static_cast<double>(stdev) < 0)
      throw std::invalid_argument("Initializer_Truncated_Normal standard deviation must be nonnegative");
  }
  void fill(std::vector<double>& a, int, int) const {
    init_detail::fill_truncated_normal(a, static_cast<double>(mean), static_cast<double>(stdev), seed);
  }
  template <class V> void fill(V const& a) const {
    init_detail::fill_view(a, [&](std::vector<double>& v) { fill(v, 0, 0); });
  }
};

namespace init_detail {
// The fan-scaled initializers: a uniform limit or a normal deviation from
// (fan_in, fan_out) (ponni_initializer.h:226-311).
template <class real, class Derived>
struct FanScaled {
  std::uint64_t seed;
  explicit FanScaled(std::uint64_t s) : seed(s) {}
  void fill(std::vector<double>& a, int fan_in, int fan_out) const {
    if (a.empty()) return;
    double const fi = fan_in, fo = fan_out;
    if (Derived::uniform) fill_uniform<real>(a, -Derived::scale(fi, fo), Derived::scale(fi, fo), seed);
    else fill_normal(a, 0.0, Derived::scale(fi, fo), seed);
  }
  template <class V> void fill(V const& a) const {
    if (a.size() == 0) return;
    double fi = 0, fo = 0;
    fans(a, fi, fo);
    fill_view(a, [&](std::vector<double>& v) { fill(v, static_cast<int>(fi), static_cast<int>(fo)); });
  }
};
}  // namespace init_detail

template <class real>
struct Initializer_Xavier_Uniform : init_detail::FanScaled<real, Initializer_Xavier_Uniform<real>> {
  static constexpr bool uniform = true;
  static double scale(double fi, double fo) { return std::sqrt(6.0 / (fi + fo)); }
  Initializer_Xavier_Uniform(std::uint64_t s = 0) : init_detail::FanScaled<real, Initializer_Xavier_Uniform>(s) {}
};
template <class real>
struct Initializer_Xavier_Normal : init_detail::FanScaled<real, Initializer_Xavier_Normal<real>> {
  static constexpr bool uniform = false;
  static double scale(double fi, double fo) { return std::sqrt(2.0 / (fi + fo)); }
  Initializer_Xavier_Normal(std::uint64_t s = 0) : init_detail::FanScaled<real, Initializer_Xavier_Normal>(s) {}
};
template <class real>
struct Initializer_He_Uniform : init_detail::FanScaled<real, Initializer_He_Uniform<real>> {
  static constexpr bool uniform = true;
  static double scale(double fi, double) { return std::sqrt(6.0 / fi); }
  Initializer_He_Uniform(std::uint64_t s = 0) : init_detail::FanScaled<real, Initializer_He_Uniform>(s) {}
};
template <class real>
struct Initializer_He_Normal : init_detail::FanScaled<real, Initializer_He_Normal<real>> {
  static constexpr bool uniform = false;
  static double scale(double fi, double) { return std::sqrt(2.0 / fi); }
  Initializer_He_Normal(std::uint64_t s = 0) : init_detail::FanScaled<real, Initializer_He_Normal>(s) {}
};
template <class real>
struct Initializer_Lecun_Uniform : init_detail::FanScaled<real, Initializer_Lecun_Uniform<real>> {
  static constexpr bool uniform = true;
  static double scale(double fi, double) { return std::sqrt(3.0 / fi); }
  Initializer_Lecun_Uniform(std::uint64_t s = 0) : init_detail::FanScaled<real, Initializer_Lecun_Uniform>(s) {}
};
template <class real>
struct Initializer_Lecun_Normal : init_detail::FanScaled<real, Initializer_Lecun_Normal<real>> {
  static constexpr bool uniform = false;
  static double scale(double fi, double) { return std::sqrt(1.0 / fi); }
  Initializer_Lecun_Normal(std::uint64_t s = 0) : init_detail::FanScaled<real, Initializer_Lecun_Normal>(s) {}
};
// Orthonormal rows or columns of a Gaussian draw, times `gain`; rank-1 arrays
// get the standard normal draw (ponni_initializer.h:313-377).
template <class real>
struct Initializer_Orthogonal {
  real gain;
  std::uint64_t seed;
  Initializer_Orthogonal(real g = real(1), std::uint64_t s = 0) : gain(g), seed(s) {
    init_detail::require_finite(static_cast<double>(gain), "Initializer_Orthogonal gain must be finite");
  }
  void fill(std::vector<double>& a, int m, int n) const {
    if (a.empty()) return;
    init_detail::fill_normal(a, 0.0, 1.0, seed);
    if (m > 0 && n > 0 && static_cast<std::size_t>(m) * n == a.size())
      init_detail::orthonormalize(a, m, n, static_cast<double>(gain));
  }
  template <class V> void fill(V const& a) const {
    require_layout_right_views<V>();
    if (a.size() == 0) return;
    init_detail::fill_view(a, [&](std::vector<double>& v) {
      if constexpr (V::rank == 2) fill(v, static_cast<int>(a.extent(0)), static_cast<int>(a.extent(1)));
      else init_detail::fill_normal(v, 0.0, 1.0, seed);
    });
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
// Each layer template takes the reference's arguments plus a trailing
// MemorySpace (src/layers/*.h), holds its parameters in Views of that space
// (`params.weights` ...), and can be rebound: rebind_memory_space<M> names the
// same layer in M, copy_to_memory_space(M) returns one holding copies of its
// Views.  A model shares its layers' Views (create_inference_model rebinds
// every layer to the model's memory space first): each forward pass reads
// them, so a write through a layer's View reaches the next pass.

namespace detail {

// Label and C-ABI descriptor of a built-in layer.
struct LayerBase {
  ponni_layer_desc desc{};
  char const* label = "";
  int get_num_inputs() const { return desc.n_in; }
  int get_num_outputs() const { return desc.n_out; }
  char const* get_label() const { return label; }
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

// Whether A looks like a view (data(), extent(), stride() and a declared
// memory space), and the element type it holds.
template <class A, class = void> struct is_view_like : std::false_type {};
template <class A>
struct is_view_like<A, std::void_t<typename A::memory_space, decltype(std::declval<A const&>().data()),
                                   decltype(std::declval<A const&>().extent(0)),
                                   decltype(std::declval<A const&>().stride(0))>> : std::true_type {};
template <class A> struct is_ponni_view : std::false_type {};
template <class D, class S> struct is_ponni_view<View<D, S>> : std::true_type {};

template <class A, class = void> struct has_call2 : std::false_type {};
template <class A>
struct has_call2<A, std::void_t<decltype(std::declval<A const&>()(0, 0)), decltype(std::declval<A const&>().extent(1))>>
    : std::true_type {};
template <class A, class = void> struct has_index : std::false_type {};
template <class A>
struct has_index<A, std::void_t<decltype(std::declval<A const&>()[0]), decltype(std::declval<A const&>().size())>>
    : std::true_type {};
// A rank-2 array argument (view or host matrix) and a rank-1 one (rank-1
// view, rank-2 view of one row or column, or a host vector).
template <class A, bool VIEW = is_view_like<A>::value> struct array_rank { static constexpr int value = 0; };
template <class A> struct array_rank<A, true> { static constexpr int value = static_cast<int>(A::rank); };
template <class A>
struct array_rank<A, false> {
  static constexpr int value = has_call2<A>::value ? 2 : has_index<A>::value ? 1 : 0;
};
template <class A>
inline constexpr bool is_array2d_v = array_rank<A>::value == 2;
template <class A>
inline constexpr bool is_array1d_v = array_rank<A>::value == 1 || (is_view_like<A>::value && array_rank<A>::value == 2);

// The elements of a view-like array (any memory space, any row stride) as
// a row-major host vector of doubles: device memory is copied, never
// dereferenced on the host.
template <class A>
std::vector<double> host_values(A const& a) {
  if constexpr (is_ponni_view<A>::value) {
    auto const h = a.copy_to_host();
    std::vector<double> out(h.size());
    for (std::size_t i = 0; i < h.size(); i++) out[i] = static_cast<double>(static_cast<float>(h[i]));
    if constexpr (std::is_same_v<typename A::non_const_value_type, double>)
      for (std::size_t i = 0; i < h.size(); i++) out[i] = h[i];
    return out;
  } else if constexpr (is_view_like<A>::value) {
    using T = std::remove_const_t<std::remove_pointer_t<decltype(a.data())>>;
    std::int64_t const rows = A::rank >= 2 ? static_cast<std::int64_t>(a.extent(0)) : 1;
    std::int64_t const cols = static_cast<std::int64_t>(A::rank >= 2 ? a.extent(1) : a.extent(0));
    std::int64_t const ld = A::rank >= 2 ? static_cast<std::int64_t>(a.stride(0)) : cols;
    std::vector<T> h(static_cast<std::size_t>(rows * cols));
    if (rows * cols > 0) {
      if constexpr (std::is_same_v<typename view_memory_space<A>::type, HostSpace>) {
        for (std::int64_t r = 0; r < rows; r++)
          for (std::int64_t c = 0; c < cols; c++) h[r * cols + c] = a.data()[r * ld + c];
      } else {
        view_check(hipMemcpy2D(h.data(), sizeof(T) * cols, a.data(), sizeof(T) * ld, sizeof(T) * cols, rows,
                               hipMemcpyDeviceToHost),
                   "hipMemcpy2D");
      }
    }
    return std::vector<double>(h.begin(), h.end());
  } else if constexpr (has_call2<A>::value) {
    std::vector<double> v(static_cast<std::size_t>(a.extent(0)) * a.extent(1));
    for (int i = 0; i < static_cast<int>(a.extent(0)); i++)
      for (int j = 0; j < static_cast<int>(a.extent(1)); j++)
        v[static_cast<std::size_t>(i) * a.extent(1) + j] = static_cast<double>(a(i, j));
    return v;
  } else {
    std::vector<double> out(a.size());
    for (std::size_t i = 0; i < out.size(); i++) out[i] = static_cast<double>(a[i]);
    return out;
  }
}

// A View<real, Space> of rank R made from values (copied in).
template <class real, class Space, int R>
auto view_from_values(char const* label, std::int64_t rows, std::int64_t cols, std::vector<double> const& v) {
  using V = std::conditional_t<R == 1, View<real*, Space>, View<real**, Space>>;
  V out;
  if constexpr (R == 1) out = V(label, cols);
  else out = V(label, rows, cols, false);
  std::vector<real> h(v.size());
  for (std::size_t i = 0; i < v.size(); i++) {
    if constexpr (std::is_same_v<real, double>) h[i] = v[i];
    else h[i] = static_cast<real>(static_cast<float>(v[i]));
  }
  out.copy_from_host(h);
  return out;
}

// The View a layer holds for a constructor argument: the argument itself when
// it is already a View of the layer's element type and memory space (or a
// foreign view of them, wrapped and kept alive), so the layer shares it;
// otherwise a copy in the layer's memory space.  R is the View's rank; a
// rank-1 View may come from a rank-2 array of one row or one column.
template <class real, class Space, int R, class A>
auto layer_view(char const* label, A const& a) {
  using V = std::conditional_t<R == 1, View<real*, Space>, View<real**, Space>>;
  if constexpr (is_view_like<A>::value) {
    std::int64_t const e0 = static_cast<std::int64_t>(a.extent(0));
    std::int64_t const e1 = A::rank >= 2 ? static_cast<std::int64_t>(a.extent(1)) : 1;
    std::int64_t const ld = A::rank >= 2 ? static_cast<std::int64_t>(a.stride(0)) : e0;
    using T = std::remove_const_t<std::remove_pointer_t<decltype(a.data())>>;
    if constexpr (std::is_same_v<T, real> && std::is_same_v<typename view_memory_space<A>::type, Space>) {
      std::shared_ptr<void> keep;
      if constexpr (is_ponni_view<A>::value) keep = a.owner();
      else keep = std::make_shared<A>(a);
      auto* p = const_cast<T*>(a.data());
      if constexpr (R == 1) {
        // rank 1, or one row, or one column (stride ld between elements)
        if (A::rank == 1 || e0 == 1) return V::wrap(p, 1, A::rank == 1 ? e0 : e1, A::rank == 1 ? e0 : e1, keep);
        if (e1 == 1 && ld == 1) return V::wrap(p, 1, e0, e0, keep);
      } else if (A::rank == 2) {
        return V::wrap(p, e0, e1, ld, keep);
      }
    }
    std::int64_t const n = e0 * e1;
    return view_from_values<real, Space, R>(label, R == 1 ? 1 : e0, R == 1 ? n : e1, host_values(a));
  } else {
    std::vector<double> v = host_values(a);
    std::int64_t rows = 1;
    if constexpr (has_call2<A>::value) rows = static_cast<std::int64_t>(a.extent(0));
    std::int64_t const cols = static_cast<std::int64_t>(v.size()) / std::max<std::int64_t>(rows, 1);
    return view_from_values<real, Space, R>(label, R == 1 ? 1 : rows, R == 1 ? static_cast<std::int64_t>(v.size()) : cols, v);
  }
}

// Write host values into a View (any space, any row stride), converted.
template <class V>
void store_values(V const& v, std::vector<double> const& values) {
  using T = typename V::non_const_value_type;
  std::vector<T> h(values.size());
  for (std::size_t i = 0; i < values.size(); i++) {
    if constexpr (std::is_same_v<T, double>) h[i] = values[i];
    else h[i] = static_cast<T>(static_cast<float>(values[i]));
  }
  v.copy_from_host(h);
}

// Trainable input of set_trainable_parameters (a View in any space or a
// host vector) as host doubles.
template <class A>
std::vector<double> trainable_values(A const& in) {
  return host_values(in);
}

}  // namespace detail

// Dense layer, W [n_in, n_out] (ponni_Matvec.h).
template <class real = float, int N_IN = 1, int N_OUT = 1, class MemorySpace = HIPSpace>
struct Matvec : detail::LayerBase {
  using memory_space = MemorySpace;
  template <class NewMemorySpace> using rebind_memory_space = Matvec<real, N_IN, N_OUT, NewMemorySpace>;
  using real1d = View<real*, MemorySpace>;
  using real2d = View<real**, MemorySpace>;
  static constexpr bool overwrite_input = false, binop = false, save = false;
  static constexpr LayerFusionKind fusion_kind = LayerFusionKind::dense;
  static constexpr int INPUT_SIZE = N_IN, OUTPUT_SIZE = N_OUT;
  struct Params {
    real2d weights;
    bool trainable = true;
  };
  Params params;

  Matvec() = default;
  template <class INIT = Initializer_Random_Uniform<real>>
  Matvec(int num_inputs, int num_outputs, bool trainable = true, INIT initializer = INIT()) {
    real2d w("Matvec_weights", num_inputs, num_outputs);
    initializer.fill(w);
    init(w, trainable);
  }
  // Weights [n_in, n_out]: a View of this element type and memory space (or a
  // foreign view of them) is shared; anything else is copied.
  template <class A, class = std::enable_if_t<detail::is_array2d_v<A>>>
  explicit Matvec(A const& weights, bool trainable = true) {
    init(detail::layer_view<real, MemorySpace, 2>("Matvec_weights", weights), trainable);
  }
  void init(real2d const& weights, bool trainable = true) {
    if (!weights.is_allocated()) abort("ERROR: Matvec weights matrix not is_allocated");
    params.weights = weights;
    params.trainable = trainable;
    desc = detail::make_desc(PONNI_LAYER_MATVEC, static_cast<int>(weights.extent(0)), static_cast<int>(weights.extent(1)));
    label = "Matvec";
  }
  template <class NewMemorySpace>
  auto copy_to_memory_space(NewMemorySpace const& space = NewMemorySpace()) const {
    return rebind_memory_space<NewMemorySpace>(create_memory_space_copy(params.weights, space), params.trainable);
  }
  using detail::LayerBase::get_num_inputs;
  using detail::LayerBase::get_num_outputs;
  static int get_num_inputs(Params const& p) { return static_cast<int>(p.weights.extent(0)); }
  static int get_num_outputs(Params const& p) { return static_cast<int>(p.weights.extent(1)); }
  int get_num_trainable_parameters() const { return params.trainable ? static_cast<int>(params.weights.size()) : 0; }
  // Consume the first get_num_trainable_parameters() values (ponni_Matvec.h:103-109).
  template <class A>
  void set_trainable_parameters(A const& in) {
    if (!params.trainable) return;
    auto v = detail::trainable_values(in);
    if (static_cast<std::int64_t>(v.size()) < params.weights.size()) abort("ERROR: Matvec trainable input too small");
    v.resize(static_cast<std::size_t>(params.weights.size()));
    detail::store_values(params.weights, v);
  }
  real1d get_trainable_parameters() const { return params.trainable ? flatten(params.weights) : real1d(); }
  // W(k, j) of the [n_in, n_out] weights, read from the View.
  double weight(int k, int j) const {
    return detail::host_values(params.weights)[static_cast<std::size_t>(k) * desc.n_out + j];
  }
  void validate() const {
    if (!params.weights.is_allocated()) abort("ERROR: weights not is_allocated");
    if (params.weights.extent(0) == 0 || params.weights.extent(1) == 0)
      abort("ERROR: Matvec weights dimensions must be nonzero");
  }
  template <class F> void for_each_segment(F&& f) const { f(0, params.weights); }
};

// Bias (ponni_Bias.h): b [n], added after the dot product.
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct Bias : detail::LayerBase {
  using memory_space = MemorySpace;
  template <class NewMemorySpace> using rebind_memory_space = Bias<real, N, NewMemorySpace>;
  using real1d = View<real*, MemorySpace>;
  static constexpr bool overwrite_input = true, binop = false, save = false;
  static constexpr LayerFusionKind fusion_kind = LayerFusionKind::pointwise;
  static constexpr int INPUT_SIZE = N, OUTPUT_SIZE = N;
  struct Params {
    real1d weights;
    bool trainable = true;
  };
  Params params;

  Bias() = default;
  template <class INIT = Initializer_Random_Uniform<real>>
  Bias(int num_inputs, bool trainable = true, INIT initializer = INIT()) {
    real1d b("Bias_weights", num_inputs);
    initializer.fill(b);
    init(b, trainable);
  }
  // b: a rank-1 View (or one row / column of a rank-2 one) of this element
  // type and memory space is shared; host vectors and other Views are copied.
  template <class A, class = std::enable_if_t<detail::is_array1d_v<A>>>
  explicit Bias(A const& weights, bool trainable = true) {
    init(detail::layer_view<real, MemorySpace, 1>("Bias_weights", weights), trainable);
  }
  void init(real1d const& weights, bool trainable = true) {
    if (!weights.is_allocated()) abort("ERROR: Bias weights not is_allocated");
    params.weights = weights;
    params.trainable = trainable;
    int const n = static_cast<int>(weights.extent(0));
    desc = detail::make_desc(PONNI_LAYER_BIAS, n, n);
    label = "Bias";
  }
  template <class NewMemorySpace>
  auto copy_to_memory_space(NewMemorySpace const& space = NewMemorySpace()) const {
    return rebind_memory_space<NewMemorySpace>(create_memory_space_copy(params.weights, space), params.trainable);
  }
  using detail::LayerBase::get_num_inputs;
  using detail::LayerBase::get_num_outputs;
  static int get_num_inputs(Params const& p) { return static_cast<int>(p.weights.extent(0)); }
  static int get_num_outputs(Params const& p) { return static_cast<int>(p.weights.extent(0)); }
  int get_num_trainable_parameters() const { return params.trainable ? static_cast<int>(params.weights.size()) : 0; }
  template <class A>
  void set_trainable_parameters(A const& in) {
    if (!params.trainable) return;
    auto v = detail::trainable_values(in);
    if (static_cast<std::int64_t>(v.size()) < params.weights.size()) abort("ERROR: Bias trainable input too small");
    v.resize(static_cast<std::size_t>(params.weights.size()));
    detail::store_values(params.weights, v);
  }
  real1d get_trainable_parameters() const { return params.trainable ? params.weights : real1d(); }
  void validate() const {
    if (!params.weights.is_allocated()) abort("ERROR: weights not is_allocated");
    if (params.weights.extent(0) == 0) abort("ERROR: Bias weights dimension must be nonzero");
  }
  template <class F> void for_each_segment(F&& f) const { f(0, params.weights); }
};

namespace detail {
// Parameter-free pointwise / barrier layers: one descriptor, rebound freely.
template <int KIND, template <class, int, class> class Self, class real, int N, class MemorySpace>
struct SimpleLayer : LayerBase {
  using memory_space = MemorySpace;
  template <class NewMemorySpace> using rebind_memory_space = Self<real, N, NewMemorySpace>;
  static constexpr bool overwrite_input = true, binop = false, save = false;
  static constexpr LayerFusionKind fusion_kind =
      (KIND == PONNI_LAYER_SOFTMAX || KIND == PONNI_LAYER_LOG_SOFTMAX || KIND == PONNI_LAYER_MIN_MAX_NORM)
          ? LayerFusionKind::barrier
          : LayerFusionKind::pointwise;
  static constexpr int INPUT_SIZE = N, OUTPUT_SIZE = N;
  struct Params {
    int num_inputs = 0;
  };
  SimpleLayer() = default;
  SimpleLayer(int n, char const* lbl, int flags = 0, double a0 = 0, double a1 = 0, double a2 = 0) {
    desc = make_desc(KIND, n, n, 0, 0, flags, a0, a1, a2);
    label = lbl;
  }
  template <class NewMemorySpace>
  auto copy_to_memory_space(NewMemorySpace const& = NewMemorySpace()) const {
    rebind_memory_space<NewMemorySpace> out;
    out.desc = desc;
    out.label = label;
    return out;
  }
  int get_num_trainable_parameters() const { return 0; }
  template <class A> void set_trainable_parameters(A const&) {}
  View<real*, MemorySpace> get_trainable_parameters() const { return {}; }
  void validate() const {
    if (desc.n_in <= 0) abort(std::string("ERROR: ") + label + " num_inputs must be > 0");
  }
  template <class F> void for_each_segment(F&&) const {}
};
}  // namespace detail

#define PONNI_SIMPLE_LAYER_BASE(NAME, KIND) detail::SimpleLayer<KIND, NAME, real, N, MemorySpace>
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct Relu : PONNI_SIMPLE_LAYER_BASE(Relu, PONNI_LAYER_RELU) {
  Relu() = default;
  explicit Relu(int n) : Relu::SimpleLayer(n, "ReLU") {}
};
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct LeakyRelu : PONNI_SIMPLE_LAYER_BASE(LeakyRelu, PONNI_LAYER_LEAKY_RELU) {
  LeakyRelu() = default;
  explicit LeakyRelu(int n, real negative_slope = real(0.01))
      : LeakyRelu::SimpleLayer(n, "LeakyReLU", 0, static_cast<double>(negative_slope)) {}
};
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct Elu : PONNI_SIMPLE_LAYER_BASE(Elu, PONNI_LAYER_ELU) {
  Elu() = default;
  explicit Elu(int n, real alpha = real(1)) : Elu::SimpleLayer(n, "ELU", 0, static_cast<double>(alpha)) {
    if (!(static_cast<double>(alpha) > 0)) abort("ERROR: ELU alpha must be > 0");
  }
};
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct Selu : PONNI_SIMPLE_LAYER_BASE(Selu, PONNI_LAYER_SELU) {
  Selu() = default;
  explicit Selu(int n) : Selu::SimpleLayer(n, "SELU") {}
};
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct Gelu : PONNI_SIMPLE_LAYER_BASE(Gelu, PONNI_LAYER_GELU) {
  Gelu() = default;
  explicit Gelu(int n, bool approximate = false)
      : Gelu::SimpleLayer(n, "GELU", approximate ? PONNI_FLAG_GELU_APPROXIMATE : 0) {}
};
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct Silu : PONNI_SIMPLE_LAYER_BASE(Silu, PONNI_LAYER_SILU) {
  Silu() = default;
  explicit Silu(int n) : Silu::SimpleLayer(n, "SiLU") {}
};
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct Sigmoid : PONNI_SIMPLE_LAYER_BASE(Sigmoid, PONNI_LAYER_SIGMOID) {
  Sigmoid() = default;
  explicit Sigmoid(int n) : Sigmoid::SimpleLayer(n, "Sigmoid") {}
};
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct Tanh : PONNI_SIMPLE_LAYER_BASE(Tanh, PONNI_LAYER_TANH) {
  Tanh() = default;
  explicit Tanh(int n) : Tanh::SimpleLayer(n, "Tanh") {}
};
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct Softplus : PONNI_SIMPLE_LAYER_BASE(Softplus, PONNI_LAYER_SOFTPLUS) {
  Softplus() = default;
  explicit Softplus(int n, real beta = real(1)) : Softplus::SimpleLayer(n, "Softplus", 0, static_cast<double>(beta)) {
    if (!(static_cast<double>(beta) > 0)) abort("ERROR: Softplus beta must be > 0");
  }
};
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct HardSigmoid : PONNI_SIMPLE_LAYER_BASE(HardSigmoid, PONNI_LAYER_HARD_SIGMOID) {
  HardSigmoid() = default;
  explicit HardSigmoid(int n, real alpha = real(0.2), real beta = real(0.5))
      : HardSigmoid::SimpleLayer(n, "HardSigmoid", 0, static_cast<double>(alpha), static_cast<double>(beta)) {}
};
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct HardSwish : PONNI_SIMPLE_LAYER_BASE(HardSwish, PONNI_LAYER_HARD_SWISH) {
  HardSwish() = default;
  explicit HardSwish(int n) : HardSwish::SimpleLayer(n, "HardSwish") {}
};
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct Mish : PONNI_SIMPLE_LAYER_BASE(Mish, PONNI_LAYER_MISH) {
  Mish() = default;
  explicit Mish(int n) : Mish::SimpleLayer(n, "Mish") {}
};
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct Softmax : PONNI_SIMPLE_LAYER_BASE(Softmax, PONNI_LAYER_SOFTMAX) {
  Softmax() = default;
  explicit Softmax(int n) : Softmax::SimpleLayer(n, "Softmax") {}
};
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct LogSoftmax : PONNI_SIMPLE_LAYER_BASE(LogSoftmax, PONNI_LAYER_LOG_SOFTMAX) {
  LogSoftmax() = default;
  explicit LogSoftmax(int n) : LogSoftmax::SimpleLayer(n, "LogSoftmax") {}
};
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct MinMaxNorm : PONNI_SIMPLE_LAYER_BASE(MinMaxNorm, PONNI_LAYER_MIN_MAX_NORM) {
  MinMaxNorm() = default;
  explicit MinMaxNorm(int n, real out_min = real(0), real out_max = real(1), real epsilon = real(1e-12))
      : MinMaxNorm::SimpleLayer(n, "MinMaxNorm", 0, static_cast<double>(out_min), static_cast<double>(out_max),
                                static_cast<double>(epsilon)) {}
};
#undef PONNI_SIMPLE_LAYER_BASE

// LayerNorm (ponni_LayerNorm.h): gamma = 1, beta = 0 by default; trainable [gamma; beta].
template <class real = float, int N = 1, class MemorySpace = HIPSpace>
struct LayerNorm : detail::LayerBase {
  using memory_space = MemorySpace;
  template <class NewMemorySpace> using rebind_memory_space = LayerNorm<real, N, NewMemorySpace>;
  using real1d = View<real*, MemorySpace>;
  static constexpr bool overwrite_input = true, binop = false, save = false;
  static constexpr int INPUT_SIZE = N, OUTPUT_SIZE = N;
  struct Params {
    real1d gamma;
    real1d beta;
    real epsilon = real(1e-5);
    bool trainable = true;
  };
  Params params;

  LayerNorm() = default;
  explicit LayerNorm(int n, real epsilon = real(1e-5), bool trainable = true) {
    real1d g("LayerNorm_gamma", n), b("LayerNorm_beta", n);
    deep_copy(g, real(1));
    init(g, b, epsilon, trainable);
  }
  template <class A, class B, class = std::enable_if_t<detail::is_array1d_v<A> && detail::is_array1d_v<B>>>
  LayerNorm(A const& gamma, B const& beta, real epsilon = real(1e-5), bool trainable = true) {
    init(detail::layer_view<real, MemorySpace, 1>("LayerNorm_gamma", gamma),
         detail::layer_view<real, MemorySpace, 1>("LayerNorm_beta", beta), epsilon, trainable);
  }
  void init(real1d const& gamma, real1d const& beta, real epsilon, bool trainable) {
    if (gamma.size() != beta.size()) abort("ERROR: LayerNorm gamma/beta sizes differ");
    if (!(static_cast<double>(epsilon) > 0)) abort("ERROR: LayerNorm epsilon must be > 0");
    params.gamma = gamma;
    params.beta = beta;
    params.epsilon = epsilon;
    params.trainable = trainable;
    int const n = static_cast<int>(gamma.extent(0));
    desc = detail::make_desc(PONNI_LAYER_LAYER_NORM, n, n, 0, 0, 0, static_cast<double>(epsilon));
    label = "LayerNorm";
  }
  template <class NewMemorySpace>
  auto copy_to_memory_space(NewMemorySpace const& space = NewMemorySpace()) const {
    return rebind_memory_space<NewMemorySpace>(create_memory_space_copy(params.gamma, space),
                                               create_memory_space_copy(params.beta, space), params.epsilon,
                                               params.trainable);
  }
  int get_num_trainable_parameters() const { return params.trainable ? static_cast<int>(2 * params.gamma.size()) : 0; }
  template <class A>
  void set_trainable_parameters(A const& in) {
    if (!params.trainable) return;
    auto v = detail::trainable_values(in);
    std::size_t const n = static_cast<std::size_t>(params.gamma.size());
    if (v.size() < 2 * n) abort("ERROR: LayerNorm trainable input too small");
    detail::store_values(params.gamma, std::vector<double>(v.begin(), v.begin() + n));
    detail::store_values(params.beta, std::vector<double>(v.begin() + n, v.begin() + 2 * n));
  }
  real1d get_trainable_parameters() const {
    if (!params.trainable) return real1d();
    auto g = detail::host_values(params.gamma), b = detail::host_values(params.beta);
    g.insert(g.end(), b.begin(), b.end());
    return detail::view_from_values<real, MemorySpace, 1>("LayerNorm_trainable", 1, static_cast<std::int64_t>(g.size()), g);
  }
  void validate() const {}
  template <class F> void for_each_segment(F&& f) const {
    f(0, params.gamma);
    f(1, params.beta);
  }
};

// Residual plumbing (ponni_Save_State.h, ponni_Binop_*.h).  ISAVE selects the
// saved-state slot, as the reference's first template argument.
template <int ISAVE, class real = float, int N = 1, class MemorySpace = HIPSpace>
struct Save_State : detail::LayerBase {
  using memory_space = MemorySpace;
  template <class NewMemorySpace> using rebind_memory_space = Save_State<ISAVE, real, N, NewMemorySpace>;
  static constexpr bool overwrite_input = true, save = true, binop = false;
  static constexpr int index = ISAVE;
  Save_State() = default;
  explicit Save_State(int n) {
    desc = detail::make_desc(PONNI_LAYER_SAVE_STATE, n, n, ISAVE);
    label = "Save_State";
  }
  template <class NewMemorySpace>
  auto copy_to_memory_space(NewMemorySpace const& = NewMemorySpace()) const {
    return rebind_memory_space<NewMemorySpace>(desc.n_in);
  }
  int get_num_trainable_parameters() const { return 0; }
  template <class A> void set_trainable_parameters(A const&) {}
  View<real*, MemorySpace> get_trainable_parameters() const { return {}; }
  void validate() const {}
  template <class F> void for_each_segment(F&&) const {}
};

template <int ISAVE, class real = float, int N = 1, class MemorySpace = HIPSpace>
struct Binop_Add : detail::LayerBase {
  using memory_space = MemorySpace;
  template <class NewMemorySpace> using rebind_memory_space = Binop_Add<ISAVE, real, N, NewMemorySpace>;
  static constexpr bool overwrite_input = true, save = false, binop = true;
  static constexpr int index = ISAVE;
  Binop_Add() = default;
  explicit Binop_Add(int n) {
    desc = detail::make_desc(PONNI_LAYER_BINOP_ADD, n, n, ISAVE);
    label = "Binop_Add";
  }
  template <class NewMemorySpace>
  auto copy_to_memory_space(NewMemorySpace const& = NewMemorySpace()) const {
    return rebind_memory_space<NewMemorySpace>(desc.n_in);
  }
  int get_num_trainable_parameters() const { return 0; }
  template <class A> void set_trainable_parameters(A const&) {}
  View<real*, MemorySpace> get_trainable_parameters() const { return {}; }
  void validate(int saved_n) const {
    if (saved_n != desc.n_in) abort("ERROR: Saved layer num inputs != this layer's num inputs");
  }
  template <class F> void for_each_segment(F&&) const {}
};

template <int ISAVE, class real = float, int N1 = 1, int N2 = 1, class MemorySpace = HIPSpace>
struct Binop_Concatenate : detail::LayerBase {
  using memory_space = MemorySpace;
  template <class NewMemorySpace> using rebind_memory_space = Binop_Concatenate<ISAVE, real, N1, N2, NewMemorySpace>;
  static constexpr bool overwrite_input = true, save = false, binop = true;
  static constexpr int index = ISAVE;
  Binop_Concatenate() = default;
  Binop_Concatenate(int num_inputs, int num_outputs, bool after = true) {
    desc = detail::make_desc(PONNI_LAYER_BINOP_CONCATENATE, num_inputs, num_outputs, ISAVE, 0,
                             after ? PONNI_FLAG_CONCAT_AFTER : 0);
    label = "Binop_Concatenate";
  }
  template <class NewMemorySpace>
  auto copy_to_memory_space(NewMemorySpace const& = NewMemorySpace()) const {
    return rebind_memory_space<NewMemorySpace>(desc.n_in, desc.n_out, (desc.flags & PONNI_FLAG_CONCAT_AFTER) != 0);
  }
  int get_num_trainable_parameters() const { return 0; }
  template <class A> void set_trainable_parameters(A const&) {}
  View<real*, MemorySpace> get_trainable_parameters() const { return {}; }
  void validate(int saved_n) const {
    if (desc.n_out != saved_n + desc.n_in)
      abort("ERROR: this layer's num outputs != this layer's num inputs + saved layer's num inputs");
  }
  template <class F> void for_each_segment(F&&) const {}
};

// out = in + (bias + W^T saved), W [NSAVE, NIN] (ponni_Binop_Projection_Add.h).
template <int ISAVE, class real = float, int NIN = 1, int NSAVE = 1, class MemorySpace = HIPSpace>
struct Binop_Projection_Add : detail::LayerBase {
  using memory_space = MemorySpace;
  template <class NewMemorySpace>
  using rebind_memory_space = Binop_Projection_Add<ISAVE, real, NIN, NSAVE, NewMemorySpace>;
  using real1d = View<real*, MemorySpace>;
  using real2d = View<real**, MemorySpace>;
  static constexpr bool overwrite_input = true, save = false, binop = true;
  static constexpr int index = ISAVE;
  struct Params {
    real2d weights;
    real1d bias;
    bool trainable = true;
  };
  Params params;

  Binop_Projection_Add() = default;
  template <class INIT = Initializer_Random_Uniform<real>>
  Binop_Projection_Add(int num_inputs, int num_saved_inputs, bool trainable = true, INIT initializer = INIT()) {
    real2d w("Binop_Projection_Add_weights", num_saved_inputs, num_inputs);
    real1d b("Binop_Projection_Add_bias", num_inputs);
    initializer.fill(w);
    initializer.fill(b);
    init(w, b, trainable);
  }
  template <class A, class B, class = std::enable_if_t<detail::is_array2d_v<A> && detail::is_array1d_v<B>>>
  Binop_Projection_Add(A const& weights, B const& bias, bool trainable = true) {
    init(detail::layer_view<real, MemorySpace, 2>("Binop_Projection_Add_weights", weights),
         detail::layer_view<real, MemorySpace, 1>("Binop_Projection_Add_bias", bias), trainable);
  }
  void init(real2d const& weights, real1d const& bias, bool trainable) {
    if (weights.extent(1) != bias.extent(0)) abort("ERROR: Binop_Projection_Add incompatible weights/bias shapes");
    params.weights = weights;
    params.bias = bias;
    params.trainable = trainable;
    desc = detail::make_desc(PONNI_LAYER_BINOP_PROJECTION_ADD, static_cast<int>(weights.extent(1)),
                             static_cast<int>(weights.extent(1)), ISAVE, static_cast<int>(weights.extent(0)));
    label = "Binop_Projection_Add";
  }
  template <class NewMemorySpace>
  auto copy_to_memory_space(NewMemorySpace const& space = NewMemorySpace()) const {
    return rebind_memory_space<NewMemorySpace>(create_memory_space_copy(params.weights, space),
                                               create_memory_space_copy(params.bias, space), params.trainable);
  }
  int get_num_trainable_parameters() const {
    return params.trainable ? static_cast<int>(params.weights.size() + params.bias.size()) : 0;
  }
  template <class A>
  void set_trainable_parameters(A const& in) {
    if (!params.trainable) return;
    auto v = detail::trainable_values(in);
    std::size_t const nw = static_cast<std::size_t>(params.weights.size()), nb = static_cast<std::size_t>(params.bias.size());
    if (v.size() < nw + nb) abort("ERROR: Binop_Projection_Add trainable input too small");
    detail::store_values(params.weights, std::vector<double>(v.begin(), v.begin() + nw));
    detail::store_values(params.bias, std::vector<double>(v.begin() + nw, v.begin() + nw + nb));
  }
  real1d get_trainable_parameters() const {
    if (!params.trainable) return real1d();
    auto w = detail::host_values(params.weights), b = detail::host_values(params.bias);
    w.insert(w.end(), b.begin(), b.end());
    return detail::view_from_values<real, MemorySpace, 1>("Binop_Projection_Add_trainable", 1,
                                                         static_cast<std::int64_t>(w.size()), w);
  }
  void validate(int saved_n) const {
    if (saved_n != desc.n_aux) abort("ERROR: saved layer size incompatible with projection weights");
  }
  template <class F> void for_each_segment(F&& f) const {
    f(0, params.weights);
    f(1, params.bias);
  }
};

// ---- the model ---------------------------------------------------------------------------

namespace detail {

template <class L>
inline constexpr bool is_builtin_v = std::is_base_of_v<LayerBase, L>;

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
  using real1d = View<real*, memory_space>;
  using real2d = View<real**, memory_space>;
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
    share_views(std::make_index_sequence<num_layers>{});
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
  // get_saved_state_size<ISAVE>() (ponni_Inference.h:204-223): the widest
  // state any Save_State<ISAVE> stores, 0 for an index no save uses.
  template <int ISAVE>
  int get_saved_state_size() const {
    static_assert(ISAVE >= 0, "saved-state index must be nonnegative");
    return ISAVE < get_num_saved_states() ? ponni_plan_saved_state_size(plan_.get(), ISAVE) : 0;
  }
  template <int REQUESTED_BUFFER>
  int get_planned_temporary_size() const {
    return REQUESTED_BUFFER == 0 ? info().tmp1_features : info().tmp2_features;
  }

  // Each layer's own validate() plus the chain check (ponni_Inference.h:719-737);
  // the plan already rejected an invalid chain, so this re-checks the layers.
  void validate() const {
    std::vector<int> saved(max_slot_index() + 1, 0);
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
  // Flattened in tuple order, in the model's memory space (ponni_Inference.h:688-716).
  real1d get_trainable_parameters() const {
    std::vector<double> v = trainable_values();
    if (v.empty()) return real1d();
    return detail::view_from_values<real, memory_space, 1>("trainable_parameters", 1,
                                                           static_cast<std::int64_t>(v.size()), v);
  }
  // Consumes get_num_trainable_parameters() values (a View in any memory space
  // or a host vector) into the layers' Views, in tuple order.
  template <class A>
  void set_trainable_parameters(A const& in) {
    std::vector<double> const v = detail::host_values(in);
    std::size_t off = 0;
    std::apply(
        [&](auto&... l) {
          auto one = [&](auto& layer) {
            if constexpr (detail::is_builtin_v<std::decay_t<decltype(layer)>>) {
              std::size_t const n = static_cast<std::size_t>(layer.get_num_trainable_parameters());
              if (n == 0) return;
              if (v.size() < off + n) abort(std::string("ERROR: ") + layer.get_label() + " trainable input too small");
              layer.set_trainable_parameters(std::vector<double>(v.begin() + off, v.begin() + off + n));
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

  // Refresh `params` (the in-kernel description, and the user layers'
  // Params of a chain that has them) from the layers' current Views.  The
  // batched forward pass reads the Views itself; in-kernel callers call this
  // after writing a layer's View directly.
  void sync() {
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
    std::vector<double> const p = trainable_values();
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
    if constexpr (has_user_layers) sync();  // their per-sample kernel reads `params`
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
  // Highest saved-state index any layer names (-1: none).
  template <class L>
  static constexpr int slot_index_of() {
    if constexpr (has_save<L>()) {
      if constexpr (L::save) return L::index;
    }
    if constexpr (has_binop<L>()) {
      if constexpr (L::binop) return L::index;
    }
    return -1;
  }
  static constexpr int max_slot_index() {
    int m = -1;
    ((m = slot_index_of<Layers>() > m ? slot_index_of<Layers>() : m), ...);
    return m;
  }
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

  // Share every built-in layer's parameter Views with the plan (the layers
  // were rebound to the model's memory space): the plan reads them at each
  // forward pass (ponni_plan_share_layer_params).
  template <std::size_t... I>
  void share_views(std::index_sequence<I...>) {
    auto one = [&](auto idx) {
      constexpr std::size_t k = decltype(idx)::value;
      using L = std::tuple_element_t<k, TUPLE>;
      if constexpr (detail::is_builtin_v<L>) {
        static_assert(std::is_same_v<typename L::memory_space, memory_space>,
                      "a model's layers live in its memory space (create_inference_model rebinds them)");
        std::get<k>(layers_).for_each_segment([&](int seg, auto const& v) {
          using V = std::decay_t<decltype(v)>;
          check(ponni_plan_share_layer_params(plan_.get(), static_cast<std::int32_t>(k), seg, v.data(),
                                              dtype_of<typename V::non_const_value_type>(), v.rows(), v.cols(),
                                              v.ld(), std::is_same_v<typename V::memory_space, HIPSpace> ? 1 : 0),
                "create_inference_model");
        });
      }
    };
    (one(std::integral_constant<std::size_t, I>{}), ...);
  }
  // Built-in layers' trainable values in tuple order, read from their Views.
  std::vector<double> trainable_values() const {
    std::vector<double> out;
    std::apply(
        [&](auto const&... l) {
          auto one = [&](auto const& layer) {
            if constexpr (detail::is_builtin_v<std::decay_t<decltype(layer)>>) {
              if (layer.get_num_trainable_parameters() == 0) return;
              auto const v = detail::host_values(layer.get_trainable_parameters());
              out.insert(out.end(), v.begin(), v.end());
            }
          };
          (one(l), ...);
        },
        layers_);
    return out;
  }

  TUPLE layers_;
  Exec exec_;
  std::shared_ptr<ponni_plan_s> plan_;
};

// ---- View copies and .ponni tensors (src/utils/ponni_view_ops.h:12-48,
// src/utils/ponni_safetensors.h:409-444) ------------------------------------------------

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
template <class L, class = void> struct has_rebind : std::false_type {};
template <class L>
struct has_rebind<L, std::void_t<typename L::memory_space, typename L::template rebind_memory_space<HostSpace>>>
    : std::true_type {};
// A layer in the model's memory space (src/ponni_create_model.h:10-18): the
// layer itself when it already lives there, so the model shares its Views;
// otherwise copy_to_memory_space.  A user layer without the rebinding
// members is used as it is.
template <class Mem, class L>
auto rebind_layer_memory_space(L const& layer, Mem const& memory_space) {
  if constexpr (!has_rebind<L>::value) {
    return layer;
  } else if constexpr (std::is_same_v<typename L::memory_space, Mem>) {
    return layer;
  } else {
    return layer.template copy_to_memory_space<Mem>(memory_space);
  }
}
template <class real, class Exec, class Mem, class... Layers>
inline auto create_model(Exec const& exec, Mem const& mem, Layers const&... layers) {
  static_assert(is_execution_space_v<Exec>, "create_inference_model requires an execution space (HIP or Host)");
  static_assert(is_memory_space_v<Mem>, "create_inference_model requires a memory space (HIPSpace or HostSpace)");
  static_assert(std::is_same_v<typename Exec::memory_space, Mem>,
                "create_inference_model execution space cannot access its memory space");
  return BasicInference<real, Exec, std::decay_t<decltype(rebind_layer_memory_space(layers, mem))>...>(
      std::make_tuple(rebind_layer_memory_space(layers, mem)...), exec);
}
}  // namespace detail

// Default model: the GPU, HIPSpace; layers in another space are copied in
// (ponni_create_model.h:40-98).  Like the reference, the default and the
// execution-space forms compute in float.
template <class First, class... Rest,
          std::enable_if_t<!is_execution_space_v<First> && !std::is_same_v<std::decay_t<First>, hipStream_t>, int> = 0>
inline auto create_inference_model(First const& first, Rest const&... rest) {
  return detail::create_model<float>(HIP(), HIPSpace(), first, rest...);
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
  return detail::create_model<float>(HIP(stream), HIPSpace(), layers...);
}
template <class... Layers>
inline auto create_inference_model_single_precision(Layers const&... layers) {
  return detail::create_model<float>(HIP(), HIPSpace(), layers...);
}
template <class... Layers>
inline auto create_inference_model_double_precision(Layers const&... layers) {
  return detail::create_model<double>(HIP(), HIPSpace(), layers...);
}
template <class... Layers>
inline auto create_inference_model_half_precision(Layers const&... layers) {
  return detail::create_model<half_t>(HIP(), HIPSpace(), layers...);
}
template <class... Layers>
inline auto create_inference_model_bhalf_precision(Layers const&... layers) {
  return detail::create_model<bhalf_t>(HIP(), HIPSpace(), layers...);
}

}  // namespace ponni
