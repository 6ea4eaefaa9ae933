// C++ facade tests (ponni_amd/include/ponni.h): the reference's own C++ unit
// tests restated against the facade.  `--cpu` runs only the checks that touch
// no device (model construction, scratch planning, parameters, fingerprints,
// .ponni files, 16-bit conversions); without it the forward passes run on
// the GPU as well.
//
// Known answers (reference files relative to its root):
//   unit/core/test_core_unit.cpp:200-221   first model -> (4, 4), no scratch
//   unit/core/test_core_unit.cpp:262-326   four fused blocks, closed form, tmp 7 / 3
//   unit/core/test_core_unit.cpp:331-378   Softmax barrier -> (tanh 1, 0), tmp 3 / 0
//   unit/core/test_core_unit.cpp:516-546   Matvec [in, out] layout -> 36, 39, 42
//   unit/core/test_core_unit.cpp:814-872   projection skip -> (5.1, 7.2, 7.8)
//   unit/core/test_template_coverage.cpp:414-500  multi-slot save -> {0,6,-2,6,-2,3}
//   unit/core/test_template_coverage.cpp:503-525  half / bhalf factories -> 5
//   unit/performance_benchmark/performance_benchmark.cpp:21-53  mean 15.4
//   unit/core/test_core_unit.cpp:380-404   host execution/memory space model -> (4, 4)
#include <cmath>
#include <cstdio>
#include <limits>
#include <stdexcept>
#include <utility>
#include <cstring>
#include <string>
#include <vector>

#include "ponni.h"

namespace {

int g_failures = 0;
int g_checks = 0;

#define CHECK(cond)                                                              \
  do {                                                                           \
    g_checks++;                                                                  \
    if (!(cond)) {                                                               \
      g_failures++;                                                              \
      std::fprintf(stderr, "FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond);     \
    }                                                                            \
  } while (0)

bool near(double a, double b, double tol) { return std::fabs(a - b) <= tol; }

template <class real>
ponni::View<real> device_matrix(int rows, int cols, std::vector<float> const& v) {
  ponni::View<real> d("x", rows, cols);
  std::vector<real> h(v.begin(), v.end());
  d.copy_from_host(h);
  return d;
}

template <class V>
std::vector<double> host(V const& v) {
  auto h = v.copy_to_host();
  return std::vector<double>(h.begin(), h.end());
}

ponni::Matrix<float> ones(int r, int c) { return ponni::Matrix<float>(r, c, 1.0f); }

// The execution space whose memory space is S (host checks build their
// layers and models in HostSpace, so they need no device).
template <class S>
using ExecOf = std::conditional_t<std::is_same_v<S, ponni::HostSpace>, ponni::Host, ponni::HIP>;

template <class S = ponni::HIPSpace>
auto four_block_model_in(ExecOf<S> const& exec = ExecOf<S>()) {
  using namespace ponni;
  return create_inference_model(
      exec, S(), Matvec<float, 1, 1, S>(ones(2, 5)), Bias<float, 1, S>(std::vector<float>(5, 0.5f)),
      Relu<float, 1, S>(5), Tanh<float, 1, S>(5), Matvec<float, 1, 1, S>(ones(5, 3)),
      Bias<float, 1, S>(std::vector<float>(3, -0.25f)), Sigmoid<float, 1, S>(3), Matvec<float, 1, 1, S>(ones(3, 7)),
      Bias<float, 1, S>(std::vector<float>(7, 0.1f)), LeakyRelu<float, 1, S>(7, 0.2f),
      Matvec<float, 1, 1, S>(ones(7, 2)), Bias<float, 1, S>(std::vector<float>(2, -0.2f)), HardSwish<float, 1, S>(2));
}
auto four_block_model() { return four_block_model_in<ponni::HIPSpace>(); }

double four_block_closed_form(double x0, double x1) {
  double const s = x0 + x1;
  double const h1 = std::tanh(std::max(0.0, s + 0.5));
  double const h2 = 1.0 / (1.0 + std::exp(-(5 * h1 - 0.25)));
  double const d3 = 3 * h2 + 0.1;
  double const h3 = d3 > 0 ? d3 : 0.2 * d3;
  double const d4 = 7 * h3 - 0.2;
  return d4 <= -3 ? 0.0 : d4 >= 3 ? d4 : d4 * (d4 + 3) / 6;
}

// ---- host-only checks ----------------------------------------------------------------

template <class S>
void test_structure_and_planning() {
  using namespace ponni;
  ExecOf<S> const ex;
  auto first = create_inference_model(ex, S(), Matvec<float, 1, 1, S>(ones(2, 2)),
                                      Bias<float, 1, S>(std::vector<float>{1, 1}), LeakyRelu<float, 1, S>(2, 0.1f));
  CHECK(first.get_num_inputs() == 2 && first.get_num_outputs() == 2);
  CHECK(first.template get_planned_temporary_size<0>() == 0 && first.template get_planned_temporary_size<1>() == 0);
  CHECK(first.get_num_fused_dense_blocks() == 1);
  auto four = four_block_model_in<S>();
  CHECK(four.template get_planned_temporary_size<0>() == 7 && four.template get_planned_temporary_size<1>() == 3);
  CHECK(four.get_num_fused_dense_blocks() == 4);
  four.validate();
  auto soft = create_inference_model(ex, S(), Matvec<float, 1, 1, S>(ones(2, 3)),
                                     Bias<float, 1, S>(std::vector<float>{0, 1, 2}), Relu<float, 1, S>(3),
                                     Softmax<float, 1, S>(3), Matvec<float, 1, 1, S>(ones(3, 2)),
                                     Bias<float, 1, S>(std::vector<float>{0, -1}), Tanh<float, 1, S>(2));
  CHECK(soft.template get_planned_temporary_size<0>() == 3 && soft.template get_planned_temporary_size<1>() == 0);
  auto res = create_inference_model(ex, S(), Save_State<0>(2), Relu<float>(2), Binop_Concatenate<0>(2, 4, true),
                                    Save_State<1>(4), Relu<float>(4), Binop_Add<1>(4),
                                    Binop_Concatenate<0>(4, 6, true));
  CHECK(res.get_num_saved_states() == 2);
  res.validate();
  // Slot indices past any fixed table: the reference takes any ISAVE and
  // sizes every slot up to the highest (ponni_Inference.h:204-223).
  auto far = create_inference_model(ex, S(), Save_State<11>(2), Relu<float>(2), Binop_Add<11>(2), Save_State<100>(2),
                                    Binop_Concatenate<100>(2, 4, false));
  CHECK(far.get_num_saved_states() == 101);
  CHECK(far.template get_saved_state_size<11>() == 2 && far.template get_saved_state_size<100>() == 2);
  CHECK(far.template get_saved_state_size<50>() == 0 && far.template get_saved_state_size<200>() == 0);
  far.validate();
}

template <class S>
void test_parameters_and_fingerprint() {
  using namespace ponni;
  ponni::Matrix<float> w(2, 3, std::vector<float>{1, 2, 3, 4, 5, 6});
  auto m = create_inference_model(ExecOf<S>(), S(), Matvec<float, 1, 1, S>(w),
                                  Bias<float, 1, S>(std::vector<float>{7, 8, 9}), Relu<float>(3),
                                  LayerNorm<float, 1, S>(3), Matvec<float, 1, 1, S>(ones(3, 1), false));
  CHECK(m.get_num_trainable_parameters() == 6 + 3 + 6);  // the last Matvec is frozen
  auto p = host(m.get_trainable_parameters());
  std::vector<double> want{1, 2, 3, 4, 5, 6, 7, 8, 9, 1, 1, 1, 0, 0, 0};
  CHECK(p == want);
  std::vector<float> q(15);
  for (int i = 0; i < 15; i++) q[i] = 0.5f * i;
  m.set_trainable_parameters(q);
  p = host(m.get_trainable_parameters());
  CHECK(std::equal(p.begin(), p.end(), q.begin()));
  CHECK(host(m.template get_layer<1>().params.weights)[0] == 3.0);
  // "ponni-template-model-v1\n" + "I\tlabel\tnin\tnout\tntrainable\n" (ponni_Inference.h:270-288)
  std::string text = "ponni-template-model-v1\n0\tMatvec\t2\t3\t6\n1\tBias\t3\t3\t3\n2\tReLU\t3\t3\t0\n"
                     "3\tLayerNorm\t3\t3\t6\n4\tMatvec\t3\t1\t0\n";
  std::string fp = ponni::ponni_fnv1a64_string(
      ponni::ponni_fnv1a64(reinterpret_cast<unsigned char const*>(text.data()), text.size()));
  CHECK(m.weight_schema_fingerprint() == fp);
}

template <class S>
void test_weights_files() {
  using namespace ponni;
  ExecOf<S> const ex;
  char const* path = "/tmp/ponni_facade_test.ponni";
  auto a = create_inference_model(ex, S(), Matvec<float, 1, 1, S>(ponni::Matrix<float>(2, 2, std::vector<float>{1, 2, 3, 4})),
                                  Bias<float, 1, S>(std::vector<float>{5, 6}));
  std::string err;
  CHECK(a.save_weights(path, &err));
  auto b = create_inference_model(ex, S(), Matvec<float, 1, 1, S>(ones(2, 2)), Bias<float, 1, S>(std::vector<float>{0, 0}));
  CHECK(b.load_weights(path, &err));
  auto p = host(b.get_trainable_parameters());
  CHECK(p.size() == 6 && p[0] == 1 && p[3] == 4 && p[5] == 6);
  auto c = create_inference_model(ex, S(), Matvec<float, 1, 1, S>(ones(2, 2)), Relu<float>(2),
                                  Bias<float, 1, S>(std::vector<float>{0, 0}));
  CHECK(!c.load_weights(path, &err));
  CHECK(err.find("fingerprint") != std::string::npos);
  auto d = create_inference_model(ex, S(), Relu<float>(2));
  CHECK(!d.load_weights(path, &err));
  CHECK(err == "cannot load weights into a model with no trainable parameters");
  CHECK(!d.save_weights(path, &err));
  CHECK(err == "cannot save weights from a model with no trainable parameters");
  auto e = detail::create_model<double>(ex, S(), Matvec<double, 1, 1, S>(ones(2, 2)),
                                        Bias<double, 1, S>(std::vector<double>{0, 0}));
  CHECK(!e.load_weights(path, &err));  // F32 file, F64 model: dtype mismatch
  std::remove(path);
}

void test_sixteen_bit_types() {
  using ponni::bhalf_t;
  using ponni::half_t;
  CHECK(half_t(1.0f).bits == 0x3c00 && half_t(-2.0f).bits == 0xc000);
  CHECK(half_t(65504.0f).bits == 0x7bff && half_t(65520.0f).bits == 0x7c00);
  CHECK(half_t(std::ldexp(1.0f, -24)).bits == 0x0001 && half_t(std::ldexp(1.0f, -25)).bits == 0x0000);
  CHECK(float(half_t(0.1f)) == 0.0999755859375f);
  CHECK(half_t(1.0f + std::ldexp(1.0f, -11)).bits == 0x3c00);       // tie to even
  CHECK(half_t(1.0f + 3 * std::ldexp(1.0f, -11)).bits == 0x3c02);   // tie to even (up)
  CHECK(bhalf_t(1.0f).bits == 0x3f80 && float(bhalf_t(3.0f)) == 3.0f);
  CHECK(float(bhalf_t(1.00390625f)) == 1.0f);  // tie to even
}

// ---- device checks -----------------------------------------------------------------------

void test_known_answers_gpu() {
  using namespace ponni;
  {  // first model
    auto m = create_inference_model(Matvec<float>(ones(2, 2)), Bias<float>(std::vector<float>{1, 1}),
                                    LeakyRelu<float>(2, 0.1f));
    auto x = device_matrix<float>(2, 1, {1, 2});
    auto y = host(m.forward_batch_parallel(x));
    CHECK(near(y[0], 4, 1e-6) && near(y[1], 4, 1e-6));
  }
  {  // Matvec layout
    auto m = create_inference_model(Matvec<float>(ponni::Matrix<float>(2, 3, std::vector<float>{10, 11, 12, 13, 14, 15})));
    auto y = host(m.forward_batch_parallel(device_matrix<float>(2, 1, {1, 2})));
    CHECK(y[0] == 36 && y[1] == 39 && y[2] == 42);
  }
  {  // four blocks
    auto m = four_block_model();
    std::vector<float> xv{1, -2, 0, 0.3f, 2, 0.5f, 0, -1};
    auto y = host(m.forward_batch_parallel(device_matrix<float>(2, 4, xv)));
    for (int b = 0; b < 4; b++) {
      double const e = four_block_closed_form(xv[b], xv[4 + b]);
      CHECK(near(y[b], e, 1e-4) && near(y[4 + b], e, 1e-4));
    }
  }
  {  // Softmax barrier
    auto m = create_inference_model(Matvec<float>(ones(2, 3)), Bias<float>(std::vector<float>{0, 1, 2}),
                                    Relu<float>(3), Softmax<float>(3), Matvec<float>(ones(3, 2)),
                                    Bias<float>(std::vector<float>{0, -1}), Tanh<float>(2));
    auto y = host(m.forward_batch_parallel(device_matrix<float>(2, 2, {0.5f, 0.5f, 0.5f, 0.5f})));
    CHECK(near(y[0], std::tanh(1.0), 1e-5) && near(y[1], std::tanh(1.0), 1e-5));
    CHECK(near(y[2], 0.0, 1e-5) && near(y[3], 0.0, 1e-5));
  }
  {  // multi-slot save
    auto m = create_inference_model(Save_State<0>(2), Relu<float>(2), Binop_Concatenate<0>(2, 4, true),
                                    Save_State<1>(4), Relu<float>(4), Binop_Add<1>(4),
                                    Binop_Concatenate<0>(4, 6, true));
    auto y = host(m.forward_batch_parallel(device_matrix<float>(2, 1, {-2, 3})));
    std::vector<double> want{0, 6, -2, 6, -2, 3};
    CHECK(y == want);
  }
  {  // projection skip
    auto m = create_inference_model(
        Save_State<0>(2), Matvec<float>(ponni::Matrix<float>(2, 3, std::vector<float>{0.25f, 0, 0, 0, 0.4f, 0.6f})),
        Binop_Projection_Add<0>(ponni::Matrix<float>(2, 3, std::vector<float>{1, 0, 0.5f, 0, 1, 0.5f}),
                                std::vector<float>{0.1f, 0.2f, 0.3f}));
    auto y = host(m.forward_batch_parallel(device_matrix<float>(2, 1, {4, 5})));
    CHECK(near(y[0], 5.1, 1e-5) && near(y[1], 7.2, 1e-5) && near(y[2], 7.8, 1e-5));
  }
  {  // performance benchmark: mean 15.4
    auto m = create_inference_model(Matvec<float>(ones(8, 8)), Bias<float>(std::vector<float>(8, 1.0f)),
                                    LeakyRelu<float>(8, 0.1f), Matvec<float>(ones(8, 8)),
                                    Bias<float>(std::vector<float>(8, 1.0f)), LeakyRelu<float>(8, 0.1f));
    int const B = 1 << 16;
    auto y = host(m.forward_batch_parallel(device_matrix<float>(8, B, std::vector<float>(8 * B, 0.1f))));
    double mean = 0;
    for (double v : y) mean += v;
    mean /= y.size();
    CHECK(near(mean, 15.4, 1e-3));
  }
  {  // half / bhalf factories: W = (2, -1), x = (3, 1) -> 5
    auto mh = create_inference_model_half_precision(Matvec<half_t>(ponni::Matrix<float>(2, 1, std::vector<float>{2, -1})));
    auto yh = host(mh.forward_batch_parallel(device_matrix<half_t>(2, 1, {3, 1})));
    CHECK(near(yh[0], 5.0, 2e-2));
    auto mb = create_inference_model_bhalf_precision(Matvec<bhalf_t>(ponni::Matrix<float>(2, 1, std::vector<float>{2, -1})));
    auto yb = host(mb.forward_batch_parallel(device_matrix<bhalf_t>(2, 1, {3, 1})));
    CHECK(near(yb[0], 5.0, 5e-2));
    auto md = create_inference_model_double_precision(Matvec<double>(ponni::Matrix<double>(2, 1, std::vector<double>{2, -1})));
    ponni::View<double> xd("x", 2, 1);
    xd.copy_from_host({3.0, 1.0});
    auto yd = host(md.forward_batch_parallel(xd));
    CHECK(yd[0] == 5.0);
  }
}

void test_views_streams_capacity_gpu() {
  using namespace ponni;
  auto m = four_block_model();
  int const B = 1000, LD = 1300;
  std::vector<float> xv(2 * LD);
  for (int i = 0; i < 2 * LD; i++) xv[i] = std::sin(0.01 * i);
  auto xw = device_matrix<float>(2, LD, xv);
  ponni::View<float> yw("y", 2, LD);
  auto x = xw.columns(100, 100 + B);  // stride(0) = 1300 > extent(1)
  auto y = yw.columns(100, 100 + B);
  hipStream_t s;
  CHECK(hipStreamCreate(&s) == hipSuccess);
  auto ms = create_inference_model(s, Matvec<float>(ones(2, 5)), Bias<float>(std::vector<float>(5, 0.5f)),
                                   Relu<float>(5), Tanh<float>(5), Matvec<float>(ones(5, 3)),
                                   Bias<float>(std::vector<float>(3, -0.25f)), Sigmoid<float>(3),
                                   Matvec<float>(ones(3, 7)), Bias<float>(std::vector<float>(7, 0.1f)),
                                   LeakyRelu<float>(7, 0.2f), Matvec<float>(ones(7, 2)),
                                   Bias<float>(std::vector<float>(2, -0.2f)), HardSwish<float>(2));
  ms.forward_batch_parallel(x, y);
  CHECK(hipStreamSynchronize(s) == hipSuccess);
  auto yh = host(yw);
  bool ok = true;
  for (int b = 0; b < LD; b++) {
    double const e = (b >= 100 && b < 100 + B) ? four_block_closed_form(xv[b], xv[LD + b]) : 0.0;
    ok = ok && near(yh[b], e, 1e-4) && near(yh[LD + b], e, 1e-4);
  }
  CHECK(ok);
  CHECK(ms.internal_state_capacity() == B);
  ms.reallocate_internal_state(0);
  CHECK(ms.internal_state_capacity() == 0);
  CHECK(hipStreamDestroy(s) == hipSuccess);
  // A write through a layer's View reaches the next forward pass (the model shares it).
  auto one = create_inference_model(Matvec<float>(ones(2, 1)));
  one.get_layer<0>().params.weights.copy_from_host({3.0f, 4.0f});
  auto r = host(one.forward_batch_parallel(device_matrix<float>(2, 1, {1, 1})));
  CHECK(r[0] == 7.0);
  (void)m;
}

// User layers under the plugin contract (unit/core/test_template_coverage.cpp:82-270):
// a fixed non-diagonal dense layer, an indexed pointwise layer and a
// feature-swapping barrier without fusion metadata.
template <class Real = float, int N = 2>
struct TestDense {
  static constexpr bool overwrite_input = false, binop = false, save = false;
  static constexpr ponni::LayerFusionKind fusion_kind = ponni::LayerFusionKind::dense;
  static constexpr int INPUT_SIZE = N, OUTPUT_SIZE = N;
  struct Params {
    int num_inputs = N;
    Real m00 = 2, m01 = 1, m10 = 1, m11 = -1;
  };
  Params params;
  char const* get_label() const { return "TestDense"; }
  int get_num_inputs() const { return params.num_inputs; }
  int get_num_outputs() const { return params.num_inputs; }
  int get_num_trainable_parameters() const { return 0; }
  void validate() const {}
  template <class InputView>
  __host__ __device__ static Real compute_output(InputView const& input, int feature, int batch, Params const& p) {
    return feature == 0 ? p.m00 * input(0, batch) + p.m01 * input(1, batch)
                        : p.m10 * input(0, batch) + p.m11 * input(1, batch);
  }
};

template <class Real = float, int N = 2>
struct TestIndexedPointwise {
  static constexpr bool overwrite_input = true, binop = false, save = false;
  static constexpr ponni::LayerFusionKind fusion_kind = ponni::LayerFusionKind::pointwise;
  static constexpr int INPUT_SIZE = N, OUTPUT_SIZE = N;
  struct Params {
    int num_inputs = N;
    Real offset = 0.5;
  };
  Params params;
  char const* get_label() const { return "TestIndexedPointwise"; }
  int get_num_inputs() const { return params.num_inputs; }
  int get_num_outputs() const { return params.num_inputs; }
  int get_num_trainable_parameters() const { return 0; }
  void validate() const {}
  __host__ __device__ static Real apply_fused(Real value, int feature, Params const& p) {
    return value + p.offset * static_cast<Real>(feature + 1);
  }
};

template <class Real = float, int N = 2>
struct TestBarrier {
  static constexpr bool overwrite_input = false, binop = false, save = false;
  static constexpr int INPUT_SIZE = N, OUTPUT_SIZE = N;
  struct Params {
    int num_inputs = N;
    Real scale = 1;
  };
  Params params;
  char const* get_label() const { return "TestBarrier"; }
  int get_num_inputs() const { return params.num_inputs; }
  int get_num_outputs() const { return params.num_inputs; }
  int get_num_trainable_parameters() const { return 0; }
  void validate() const {}
  template <class InputView, class OutputView>
  __host__ __device__ static void compute_all_outputs(InputView const& input, OutputView const& output, int batch,
                                                      Params const& p) {
    output(0, batch) = p.scale * input(1, batch);
    output(1, batch) = p.scale * input(0, batch);
  }
};

// A binop user layer: out = in * saved (reads saved state ISAVE).
template <int ISAVE, class Real = float, int N = 2>
struct TestMultiplySaved {
  static constexpr bool overwrite_input = true, binop = true, save = false;
  static constexpr int index = ISAVE;
  static constexpr int INPUT_SIZE = N, OUTPUT_SIZE = N;
  struct Params {
    int num_inputs = N;
  };
  Params params;
  char const* get_label() const { return "TestMultiplySaved"; }
  int get_num_inputs() const { return params.num_inputs; }
  int get_num_outputs() const { return params.num_inputs; }
  int get_num_trainable_parameters() const { return 0; }
  void validate(int) const {}
  template <class InputView, class SavedView, class OutputView>
  __host__ __device__ static void compute_all_outputs(InputView const& input, SavedView const& saved,
                                                      OutputView const& output, int batch, Params const& p) {
    for (int f = 0; f < p.num_inputs; f++) output(f, batch) = input(f, batch) * saved(f, batch);
  }
};

void test_user_layers_cpu() {
  using namespace ponni;
  static_assert(LayerTraits<TestBarrier<float, 2>>::fusion_kind == LayerFusionKind::barrier);
  static_assert(is_dense_layer_v<TestDense<float, 2>>);
  static_assert(is_pointwise_layer_v<TestIndexedPointwise<float, 2>>);
  static_assert(is_dense_layer_v<Matvec<float>> && is_pointwise_layer_v<Relu<float>> &&
                LayerTraits<Softmax<float>>::fusion_kind == LayerFusionKind::barrier);
  using Model = decltype(create_inference_model(TestDense<float, 2>(), TestIndexedPointwise<float, 2>(),
                                                TestBarrier<float, 2>(), TestDense<float, 2>()));
  static_assert(Model::has_user_layers && Model::get_num_fused_dense_blocks() == 2);
  auto m = create_inference_model(TestDense<float, 2>(), TestIndexedPointwise<float, 2>(), TestBarrier<float, 2>(),
                                  TestDense<float, 2>());
  CHECK(m.get_num_inputs() == 2 && m.get_num_outputs() == 2 && m.get_num_trainable_parameters() == 0);
}

// Host execution-space models (test_core_unit.cpp:380-404): the same
// chains on the host, through the library's host executor or, with user
// layers, the per-sample interpreter on the host.
void test_host_models_cpu() {
  using namespace ponni;
  {  // test_core_unit.cpp:380-404
    auto host_model = create_inference_model(DefaultHostExecutionSpace(), HostSpace(),
                                             Matvec<float, 1, 1, HostSpace>(ones(2, 2)),
                                             Bias<float, 1, HostSpace>(std::vector<float>(2, 1.0f)),
                                             LeakyRelu<float>(2, 0.1f));
    static_assert(std::is_same_v<typename decltype(host_model)::execution_space, DefaultHostExecutionSpace>);
    static_assert(std::is_same_v<typename decltype(host_model)::memory_space, HostSpace>);
    static_assert(std::is_same_v<typename decltype(create_inference_model(Relu<float>(2)))::memory_space, HIPSpace>);
    View<float, HostSpace> host_input("host_input", 2, 1), host_output("host_output", 2, 1);
    host_input(0, 0) = 1.0f;
    host_input(1, 0) = 2.0f;
    host_model.forward_batch_parallel(host_input, host_output);
    CHECK(near(host_output(0, 0), 4.0, 1e-6) && near(host_output(1, 0), 4.0, 1e-6));
  }
  {  // the four-block closed form over a batch, 3 host threads, strided views
    auto m = four_block_model_in<HostSpace>(Host(3));
    int const B = 1000;
    View<float, HostSpace> x("x", 2, B + 7);
    for (int b = 0; b < B; b++) {
      x(0, b) = std::sin(0.1f * b);
      x(1, b) = std::cos(0.3f * b);
    }
    auto y = m.forward_batch_parallel(x.columns(0, B));
    static_assert(std::is_same_v<typename decltype(y)::memory_space, HostSpace>);
    bool ok = true;
    for (int b = 0; b < B; b++)
      for (int o = 0; o < 2; o++) ok = ok && near(y(o, b), four_block_closed_form(x(0, b), x(1, b)), 2e-5);
    CHECK(ok);
    // one sample through the in-kernel form, here called on the host
    SArray<float, 2> in;
    SArray<float, 2> out;
    in(0) = 0.25f;
    in(1) = -0.5f;
    decltype(m)::forward_batch_parallel_in_kernel(in, out, m.params);
    CHECK(near(out(0), four_block_closed_form(0.25, -0.5), 2e-5) && near(out(1), out(0), 0.0));
  }
  {  // user layers on the host: test_template_coverage.cpp:740-790 -> (4.5, -4.5), and a mixed chain
    auto m = create_inference_model(Host(), TestDense<float, 2>(), TestIndexedPointwise<float, 2>(),
                                    TestBarrier<float, 2>(), TestDense<float, 2>());
    View<float, HostSpace> x("x", 2, 1);
    x(0, 0) = 1.0f;
    x(1, 0) = 2.0f;
    auto y = m.forward_batch_parallel(x);
    CHECK(near(y(0, 0), 4.5, 1e-6) && near(y(1, 0), -4.5, 1e-6));
    Matrix<float> w(2, 2, std::vector<float>{0.5f, -1.0f, 2.0f, 0.25f});
    auto mixed = create_inference_model(Host(), HostSpace(), Matvec<float, 1, 1, HostSpace>(w),
                                        Bias<float, 1, HostSpace>(std::vector<float>{0.1f, -0.2f}),
                                        TestIndexedPointwise<float, 2>(),
                                        Save_State<0>(2), Relu<float>(2), TestBarrier<float, 2>(),
                                        TestMultiplySaved<0, float, 2>(), Binop_Add<0>(2), Tanh<float>(2));
    int const B = 300;
    View<float, HostSpace> xs("xs", 2, B);
    for (int i = 0; i < 2 * B; i++) xs(i / B, i % B) = std::sin(0.37f * i) * 2.0f;
    auto ys = mixed.forward_batch_parallel(xs);
    bool ok = true;
    for (int b = 0; b < B; b++) {
      double const x0 = xs(0, b), x1 = xs(1, b);
      double const d0 = 0.5 * x0 + 2.0 * x1 + 0.1 + 0.5;
      double const d1 = -1.0 * x0 + 0.25 * x1 - 0.2 + 1.0;
      double const r0 = std::max(0.0, d0), r1 = std::max(0.0, d1);
      double const m0 = r1 * d0 + d0, m1 = r0 * d1 + d1;
      ok = ok && near(ys(0, b), std::tanh(m0), 2e-5) && near(ys(1, b), std::tanh(m1), 2e-5);
    }
    CHECK(ok);
  }
  {  // an F64 host model; parameter updates reach it
    auto m = detail::create_model<double>(Host(), HostSpace(), Matvec<double, 1, 1, HostSpace>(Matrix<double>(3, 2, 1.0)),
                                          LeakyRelu<double>(2, 0.1));
    View<double, HostSpace> x("x", 3, 2);
    x(0, 0) = 1.0;
    x(1, 0) = 2.0;
    x(2, 0) = -4.5;
    x(0, 1) = x(1, 1) = x(2, 1) = 1.0;
    auto y = m.forward_batch_parallel(x);
    CHECK(y(0, 0) == -0.1 * 1.5 && y(1, 0) == -0.1 * 1.5 && y(0, 1) == 3.0);
    m.set_trainable_parameters(std::vector<double>(6, 2.0));
    y = m.forward_batch_parallel(x);
    CHECK(y(0, 0) == -0.1 * 3.0 && y(1, 1) == 6.0);
  }
}

template <class Model>
__global__ void in_kernel_sarray2(typename Model::Params p, float* result) {
  ponni::SArray<float, 2> in;
  ponni::SArray<float, 2> out;
  in(0) = 1.0f;
  in(1) = 2.0f;
  Model::forward_batch_parallel_in_kernel(in, out, p);
  result[0] = out(0);
  result[1] = out(1);
}

void test_user_layers_gpu() {
  using namespace ponni;
  {  // test_template_coverage.cpp:740-790: dense, indexed pointwise, barrier, dense -> (4.5, -4.5)
    auto m = create_inference_model(TestDense<float, 2>(), TestIndexedPointwise<float, 2>(), TestBarrier<float, 2>(),
                                    TestDense<float, 2>());
    auto y = host(m.forward_batch_parallel(device_matrix<float>(2, 1, {1, 2})));
    CHECK(near(y[0], 4.5, 1e-6) && near(y[1], -4.5, 1e-6));
    View<float> r("r", 1, 2);
    using M = decltype(m);
    hipLaunchKernelGGL((in_kernel_sarray2<M>), dim3(1), dim3(1), 0, 0, m.params, r.data());
    CHECK(hipDeviceSynchronize() == hipSuccess);
    auto h = host(r);
    CHECK(near(h[0], 4.5, 1e-6) && near(h[1], -4.5, 1e-6));
  }
  {  // user layers among built-in ones, saved states included, over a batch
    Matrix<float> w(2, 2, std::vector<float>{0.5f, -1.0f, 2.0f, 0.25f});
    auto m = create_inference_model(Matvec<float>(w), Bias<float>(std::vector<float>{0.1f, -0.2f}),
                                    TestIndexedPointwise<float, 2>(), Save_State<0>(2), Relu<float>(2),
                                    TestBarrier<float, 2>(), TestMultiplySaved<0, float, 2>(), Binop_Add<0>(2),
                                    Tanh<float>(2));
    int const B = 1000;
    std::vector<float> xv(2 * B);
    for (int i = 0; i < 2 * B; i++) xv[i] = std::sin(0.37f * i) * 2.0f;
    auto y = host(m.forward_batch_parallel(device_matrix<float>(2, B, xv)));
    for (int b = 0; b < B; b++) {
      double const x0 = xv[b], x1 = xv[B + b];
      double const d0 = 0.5 * x0 + 2.0 * x1 + 0.1 + 0.5;
      double const d1 = -1.0 * x0 + 0.25 * x1 - 0.2 + 1.0;
      double const r0 = std::max(0.0, d0), r1 = std::max(0.0, d1);
      double const s0 = r1, s1 = r0;                    // barrier swaps
      double const m0 = s0 * d0 + d0, m1 = s1 * d1 + d1;  // * saved, + saved
      CHECK(near(y[b], std::tanh(m0), 2e-5) && near(y[B + b], std::tanh(m1), 2e-5));
    }
  }
}

// In-kernel inference (ponni_Inference.h:394-408, :592-665): application
// kernels evaluating samples with the model's `params`.
template <class Model, class In, class Out>
__global__ void in_kernel_views(In in, Out out, typename Model::Params p, int n) {
  int const b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < n) Model::forward_batch_parallel_in_kernel(in, out, p, b);
}

template <class Model>
__global__ void in_kernel_sarray(typename Model::Params p, float* result) {
  ponni::SArray<float, 2> in;
  ponni::SArray<float, 1> out;
  in(0) = 1.0f;
  in(1) = 2.0f;
  Model::forward_batch_parallel_in_kernel(in, out, p);
  result[0] = out(0);
}

// unit/core/test_core_unit.cpp:1019-1069: TwoHalf / TwoMask lanes.  The 16
// results of the reference test, computed where `two_half_lanes` runs.
__host__ __device__ inline void two_half_lanes(float* r) {
  using ponni::TwoHalf;
  using ponni::TwoMask;
  TwoHalf const left = TwoHalf::from_floats(2.0f, -3.0f);
  TwoHalf const right = TwoHalf::from_floats(4.0f, 5.0f);
  TwoHalf const added = left + right;
  TwoHalf const fused = TwoHalf::fma(left, right, TwoHalf::from_floats(1.0f, 2.0f));
  TwoHalf const rounded_even = TwoHalf::round(TwoHalf::from_floats(2.5f, -3.5f));
  TwoHalf const rounded_odd = TwoHalf::round(TwoHalf::from_floats(1.5f, -2.5f));
  TwoHalf const signs = TwoHalf::sign(TwoHalf::from_floats(__builtin_nanf(""), -0.0f));
  TwoMask const greater = TwoHalf::greater(left, right);
  TwoMask const either = TwoMask::logical_or(greater, TwoMask::from_bools(true, false));
  TwoMask const inverted = TwoMask::logical_not(either);
  TwoHalf const selected = TwoHalf::select(inverted, left, right);
  float const v[16] = {added.low(),        added.high(),       fused.low(),       fused.high(),
                       rounded_even.low(), rounded_even.high(), rounded_odd.low(), rounded_odd.high(),
                       signs.low(),        signs.high(),       greater.low() ? 1.0f : 0.0f, greater.high() ? 1.0f : 0.0f,
                       inverted.low() ? 1.0f : 0.0f, inverted.high() ? 1.0f : 0.0f, selected.low(), selected.high()};
  for (int i = 0; i < 16; i++) r[i] = v[i];
}

__global__ void two_half_kernel(float* r) { two_half_lanes(r); }

void check_two_half_lanes(float const* r) {
  CHECK(r[0] == 6.0f && r[1] == 2.0f && r[2] == 9.0f && r[3] == -13.0f);
  CHECK(r[4] == 2.0f && r[5] == -4.0f && r[6] == 2.0f && r[7] == -2.0f);  // ties to even
  CHECK(std::isnan(r[8]) && r[9] == 0.0f && !std::signbit(r[9]));          // sign(NaN), sign(-0) = +0
  CHECK(r[10] == 0.0f && r[11] == 0.0f && r[12] == 0.0f && r[13] == 1.0f);
  CHECK(r[14] == 4.0f && r[15] == -3.0f);
}

void test_two_half_cpu() {
  float r[16];
  two_half_lanes(r);
  check_two_half_lanes(r);
  using ponni::TwoHalf;
  // one rounding per lane: 2^-11 * (1 + 2^-10) * (1 - 2^-10) + (1 + 2^-10) is
  // exactly (1 + 2^-10) + 2^-11 - 2^-31, just below the midpoint, so it
  // rounds down to 1 + 2^-10 (two roundings would tie to 1 + 2^-9).
  TwoHalf const a = TwoHalf::splat(static_cast<_Float16>(std::ldexp(1.0f + std::ldexp(1.0f, -10), -11)));
  TwoHalf const b = TwoHalf::splat(static_cast<_Float16>(1.0f - std::ldexp(1.0f, -10)));
  TwoHalf const c = TwoHalf::splat(static_cast<_Float16>(1.0f + std::ldexp(1.0f, -10)));
  CHECK(TwoHalf::fma(a, b, c).low() == 1.0f + std::ldexp(1.0f, -10));
  // activations in fp32 per lane, rounded once; predicates
  TwoHalf const x = TwoHalf::from_floats(0.5f, -1.25f);
  CHECK(TwoHalf::tanh(x).low() == static_cast<float>(static_cast<_Float16>(std::tanh(0.5f))));
  CHECK(TwoHalf::relu(x).high() == 0.0f && TwoHalf::leaky_relu(x, 0.5f).high() == -0.625f);
  CHECK(TwoHalf::maximum(x, TwoHalf::zero()).low() == 0.5f && TwoHalf::minimum(x, TwoHalf::zero()).high() == -1.25f);
  TwoHalf const inf = TwoHalf::from_floats(-INFINITY, INFINITY);
  CHECK(!TwoHalf::is_inf(inf, false, true).low() && TwoHalf::is_inf(inf, false, true).high());
  CHECK(TwoHalf::is_nan(TwoHalf::from_floats(__builtin_nanf(""), 1.0f)).low());
  CHECK(ponni::TwoMask::equal(ponni::TwoMask::splat(true), ponni::TwoMask::from_bools(true, false)).low());
  CHECK(sizeof(TwoHalf) == sizeof(__half2) && sizeof(ponni::TwoMask) == 1);
}

void test_two_half_gpu() {
  float* d = nullptr;
  CHECK(hipMalloc(&d, 16 * sizeof(float)) == hipSuccess);
  hipLaunchKernelGGL(two_half_kernel, dim3(1), dim3(1), 0, 0, d);
  float r[16];
  CHECK(hipMemcpy(r, d, sizeof r, hipMemcpyDeviceToHost) == hipSuccess);
  check_two_half_lanes(r);
  CHECK(hipFree(d) == hipSuccess);
}

void test_in_kernel_gpu() {
  using namespace ponni;
  {  // unit/core/test_core_unit.cpp:280-322: the four-block model, batch and in-kernel agree
    auto m = four_block_model();
    std::vector<float> xv{1, -2, 0, 0.3f, 2, 0.5f, 0, -1};
    auto x = device_matrix<float>(2, 4, xv);
    auto yb = host(m.forward_batch_parallel(x));
    View<float> yk("yk", 2, 4);
    auto const params = m.params;
    using M = decltype(m);
    hipLaunchKernelGGL((in_kernel_views<M, DeviceView<float>, DeviceView<float>>), dim3(1), dim3(64), 0, 0,
                       x.device(), yk.device(), params, 4);
    CHECK(hipDeviceSynchronize() == hipSuccess);
    auto y = host(yk);
    for (int i = 0; i < 8; i++) CHECK(near(y[i], yb[i], 1e-5));
    for (int b = 0; b < 4; b++) CHECK(near(y[b], four_block_closed_form(xv[b], xv[4 + b]), 1e-4));
  }
  {  // unit/core/test_template_coverage.cpp:359-384: SArray form -> 6
    auto m = create_inference_model(Matvec<float, 2, 2>(Matrix<float>(2, 2, std::vector<float>{1, 2, 3, 4})),
                                    Bias<float, 2>(std::vector<float>{0.5f, -1.0f}), Relu<float, 2>(2),
                                    Matvec<float, 2, 1>(Matrix<float>(2, 1, std::vector<float>{2, -1})));
    View<float> r("r", 1, 1);
    using M = decltype(m);
    hipLaunchKernelGGL((in_kernel_sarray<M>), dim3(1), dim3(1), 0, 0, m.params, r.data());
    CHECK(hipDeviceSynchronize() == hipSuccess);
    CHECK(near(host(r)[0], 6.0, 1e-6));
  }
  {  // saved states and a projection skip (test_template_coverage.cpp:414-500), strided columns
    auto m = create_inference_model(Save_State<0>(2), Relu<float>(2), Binop_Concatenate<0>(2, 4, true),
                                    Save_State<1>(4), Relu<float>(4), Binop_Add<1>(4),
                                    Binop_Concatenate<0>(4, 6, true));
    View<float> xs("xs", 2, 5);
    xs.copy_from_host(std::vector<float>{-2, 0, 0, 0, 0, 3, 0, 0, 0, 0});
    auto x = xs.columns(0, 1);
    View<float> ys("ys", 6, 3);
    auto y = ys.columns(0, 1);
    using M = decltype(m);
    hipLaunchKernelGGL((in_kernel_views<M, DeviceView<float>, DeviceView<float>>), dim3(1), dim3(64), 0, 0,
                       x.device(), y.device(), m.params, 1);
    CHECK(hipDeviceSynchronize() == hipSuccess);
    auto h = host(ys);
    std::vector<double> want{0, 6, -2, 6, -2, 3};
    for (int f = 0; f < 6; f++) CHECK(h[f * 3] == want[f]);
  }
  {  // a parameter change reaches `params`
    auto m = create_inference_model(Matvec<float>(ones(2, 2)), Bias<float>(std::vector<float>{1, 1}));
    auto x = device_matrix<float>(2, 1, {1, 2});
    auto p = host(m.get_trainable_parameters());
    for (auto& v : p) v *= 2.0;
    m.set_trainable_parameters(p);
    View<float> yk("yk", 2, 1);
    using M = decltype(m);
    hipLaunchKernelGGL((in_kernel_views<M, DeviceView<float>, DeviceView<float>>), dim3(1), dim3(64), 0, 0,
                       x.device(), yk.device(), m.params, 1);
    CHECK(hipDeviceSynchronize() == hipSuccess);
    auto y = host(yk);
    CHECK(near(y[0], 8.0, 1e-6) && near(y[1], 8.0, 1e-6));
  }
}

// ---- initializers (unit/core/test_core_unit.cpp:874-1017) --------------------------------

struct Stats {
  double minimum, maximum, mean, variance;
};
template <class V>
Stats stats_of(V const& v) {
  auto h = host(v);
  Stats s{h[0], h[0], 0, 0};
  for (double x : h) {
    s.minimum = std::min(s.minimum, x);
    s.maximum = std::max(s.maximum, x);
    s.mean += x;
  }
  s.mean /= h.size();
  for (double x : h) s.variance += (x - s.mean) * (x - s.mean);
  s.variance /= h.size();
  return s;
}
template <class Init>
bool throws_invalid(Init make) {
  try {
    make();
  } catch (std::invalid_argument const&) {
    return true;
  }
  return false;
}

void test_initializers_cpu() {
  using namespace ponni;
  using real2d = View<float**, HostSpace>;
  int constexpr fan_in = 512, fan_out = 384;
  real2d values("initializer_values", fan_in, fan_out), repeated("initializer_repeated", fan_in, fan_out);
  auto variance_ok = [](Stats const& s, double expected) { return std::fabs(s.variance - expected) / expected < 0.05; };
  auto fill_twice = [&](auto const& init) {
    init.fill(values);
    init.fill(repeated);
    CHECK(host(values) == host(repeated));  // deterministic for a nonzero seed
    return stats_of(values);
  };
  Initializer_Zeros<float>().fill(values);
  auto st = stats_of(values);
  CHECK(st.minimum == 0.0 && st.maximum == 0.0);
  Initializer_Ones<float>().fill(values);
  st = stats_of(values);
  CHECK(st.minimum == 1.0 && st.maximum == 1.0);
  Initializer_Constant<float>(2.5f).fill(values);
  st = stats_of(values);
  CHECK(st.minimum == 2.5 && st.maximum == 2.5);
  st = fill_twice(Initializer_Random_Uniform<float>(-0.2f, 0.3f, 111));
  CHECK(st.minimum >= -0.2 && st.maximum < 0.3 && std::fabs(st.mean - 0.05) < 0.005);
  CHECK(variance_ok(st, 0.25 / 12.0));
  st = fill_twice(Initializer_Random_Normal<float>(0.35f, 0.4f, 222));
  CHECK(std::fabs(st.mean - 0.35) < 0.01 && variance_ok(st, 0.16));
  st = fill_twice(Initializer_Truncated_Normal<float>(-0.2f, 0.3f, 333));
  CHECK(st.minimum >= -0.8 && st.maximum <= 0.4 && std::fabs(st.mean + 0.2) < 0.01);
  CHECK(variance_ok(st, 0.09 * 0.7737413));  // two-sigma truncation: 1 - 4 phi(2) / (2 Phi(2) - 1)
  double const xv = 2.0 / (fan_in + fan_out), hv = 2.0 / fan_in, lv = 1.0 / fan_in;
  st = fill_twice(Initializer_Xavier_Uniform<float>(444));
  double const xl = std::sqrt(6.0 / (fan_in + fan_out));
  CHECK(st.minimum >= -xl && st.maximum < xl && variance_ok(st, xv));
  CHECK(variance_ok(fill_twice(Initializer_Xavier_Normal<float>(555)), xv));
  st = fill_twice(Initializer_He_Uniform<float>(666));
  double const hl = std::sqrt(6.0 / fan_in);
  CHECK(st.minimum >= -hl && st.maximum < hl && variance_ok(st, hv));
  CHECK(variance_ok(fill_twice(Initializer_He_Normal<float>(777)), hv));
  st = fill_twice(Initializer_Lecun_Uniform<float>(888));
  double const ll = std::sqrt(3.0 / fan_in);
  CHECK(st.minimum >= -ll && st.maximum < ll && variance_ok(st, lv));
  CHECK(variance_ok(fill_twice(Initializer_Lecun_Normal<float>(999)), lv));
  // Orthogonal: orthonormal columns of a tall array, rows of a wide one, times the gain.
  for (auto [m, n] : {std::pair<int, int>{48, 16}, {16, 48}}) {
    View<double**, HostSpace> q("q", m, n);
    Initializer_Orthogonal<double>(2.0, 1234).fill(q);
    int const k = std::min(m, n);
    bool ortho = true;
    for (int a = 0; a < k; a++)
      for (int b = 0; b < k; b++) {
        double dot = 0;
        for (int i = 0; i < std::max(m, n); i++) dot += m >= n ? q(i, a) * q(i, b) : q(a, i) * q(b, i);
        ortho = ortho && std::fabs(dot - (a == b ? 4.0 : 0.0)) < 1e-9;
      }
    CHECK(ortho);
  }
  // zero-size Views are no-op targets for every initializer
  real2d empty("initializer_empty", 0, fan_out);
  Initializer_None<float>().fill(empty);
  Initializer_Zeros<float>().fill(empty);
  Initializer_Random_Uniform<float>(-1.0f, 1.0f, 1).fill(empty);
  Initializer_Random_Normal<float>(0.0f, 1.0f, 2).fill(empty);
  Initializer_Truncated_Normal<float>(0.0f, 1.0f, 3).fill(empty);
  Initializer_Xavier_Uniform<float>(4).fill(empty);
  Initializer_Xavier_Normal<float>(5).fill(empty);
  Initializer_He_Uniform<float>(6).fill(empty);
  Initializer_He_Normal<float>(7).fill(empty);
  Initializer_Lecun_Uniform<float>(8).fill(empty);
  Initializer_Lecun_Normal<float>(9).fill(empty);
  Initializer_Orthogonal<float>(1.0f, 10).fill(empty);
  CHECK(empty.size() == 0);
  // degenerate distributions fill their exact value
  Initializer_Random_Uniform<float>(0.75f, 0.75f, 11).fill(values);
  st = stats_of(values);
  CHECK(st.minimum == 0.75 && st.maximum == 0.75);
  Initializer_Random_Normal<float>(-0.5f, 0.0f, 12).fill(values);
  st = stats_of(values);
  CHECK(st.minimum == -0.5 && st.maximum == -0.5);
  Initializer_Truncated_Normal<float>(0.25f, 0.0f, 13).fill(values);
  st = stats_of(values);
  CHECK(st.minimum == 0.25 && st.maximum == 0.25);
  // None leaves values alone
  Initializer_Constant<float>(3.0f).fill(values);
  Initializer_None<float>().fill(values);
  CHECK(stats_of(values).maximum == 3.0);
  float const inf = std::numeric_limits<float>::infinity(), nan = std::numeric_limits<float>::quiet_NaN();
  CHECK(throws_invalid([] { Initializer_Random_Uniform<float>(1.0f, -1.0f, 1); }));
  CHECK(throws_invalid([&] { Initializer_Random_Uniform<float>(nan, 1.0f, 1); }));
  CHECK(throws_invalid([&] { Initializer_Random_Uniform<float>(0.0f, inf, 1); }));
  CHECK(throws_invalid([] { Initializer_Random_Normal<float>(0.0f, -1.0f, 1); }));
  CHECK(throws_invalid([&] { Initializer_Random_Normal<float>(nan, 1.0f, 1); }));
  CHECK(throws_invalid([&] { Initializer_Random_Normal<float>(0.0f, inf, 1); }));
  CHECK(throws_invalid([] { Initializer_Truncated_Normal<float>(0.0f, -1.0f, 1); }));
  CHECK(throws_invalid([&] { Initializer_Truncated_Normal<float>(nan, 1.0f, 1); }));
  CHECK(throws_invalid([&] { Initializer_Truncated_Normal<float>(0.0f, inf, 1); }));
  CHECK(throws_invalid([&] { Initializer_Orthogonal<float>(inf, 1); }));
  CHECK(throws_invalid([&] { Initializer_Orthogonal<float>(nan, 1); }));
  // layer constructors take any initializer (ponni_Matvec.h:38-44)
  Matvec<float, 1, 1, HostSpace> mv(6, 4, true, Initializer_Orthogonal<float>(1.0f, 7));
  Bias<float, 1, HostSpace> bv(4, true, Initializer_Lecun_Normal<float>(8));
  CHECK(mv.get_num_inputs() == 6 && mv.get_num_outputs() == 4 && bv.get_num_inputs() == 4);
  Matvec<float, 1, 1, HostSpace> cv(2, 3, true, Initializer_Constant<float>(2.0f));
  auto cw = host(cv.params.weights);
  CHECK(cw.size() == 6 && cw[0] == 2.0 && cw[5] == 2.0);
}

// ---- layer Views, memory spaces and rebinding (ponni_create_model.h:10-18) -----------------

void test_rebinding_cpu() {
  using namespace ponni;
  View<float**, HostSpace> w("w", 2, 3);
  for (int i = 0; i < 6; i++) w(i / 3, i % 3) = 1.0f + i;
  Matvec<float, 1, 1, HostSpace> mv(w, true);
  static_assert(std::is_same_v<Matvec<float>::rebind_memory_space<HostSpace>, Matvec<float, 1, 1, HostSpace>>);
  static_assert(std::is_same_v<Matvec<float>::memory_space, HIPSpace>);
  CHECK(mv.params.weights.data() == w.data());  // the layer holds the caller's View
  using HostMatvec = Matvec<float, 1, 1, HostSpace>;
  CHECK(HostMatvec::get_num_inputs(mv.params) == 2 && mv.get_num_outputs() == 3);
  // set_trainable_parameters writes into the View (test_core_unit.cpp:530-538)
  View<float*, HostSpace> fresh("fresh", 6);
  for (int i = 0; i < 6; i++) fresh(i) = 10.0f + i;
  mv.set_trainable_parameters(fresh);
  CHECK(w(0, 0) == 10.0f && w(1, 2) == 15.0f);
  auto got = host(mv.get_trainable_parameters());
  CHECK(got.size() == 6 && got[0] == 10.0 && got[5] == 15.0);
  // a host model shares the layer's View: a later write through it is seen
  auto m = create_inference_model(Host(1), HostSpace(), mv);
  View<float, HostSpace> x("x", 2, 1), y("y", 3, 1);
  x(0, 0) = 1.0f;
  x(1, 0) = 2.0f;
  m.forward_batch_parallel(x, y);
  CHECK(y(0, 0) == 36.0f && y(1, 0) == 39.0f && y(2, 0) == 42.0f);
  w(0, 0) = 0.0f;
  m.forward_batch_parallel(x, y);
  CHECK(y(0, 0) == 26.0f);
  // copy_to_memory_space gives an independent copy
  auto copy = mv.copy_to_memory_space<HostSpace>();
  static_assert(std::is_same_v<decltype(copy), Matvec<float, 1, 1, HostSpace>>);
  CHECK(copy.params.weights.data() != w.data() && host(copy.params.weights) == host(w));
  w(1, 1) = -7.0f;
  CHECK(host(copy.params.weights)[4] == 14.0);
  // LayerNorm and Projection_Add hold two Views each
  View<float*, HostSpace> g("g", 3), b("b", 3);
  deep_copy(g, 2.0f);
  LayerNorm<float, 1, HostSpace> ln(g, b);
  CHECK(ln.params.gamma.data() == g.data() && ln.get_num_trainable_parameters() == 6);
  Binop_Projection_Add<0, float, 1, 1, HostSpace> pa(Matrix<float>(2, 3, 0.5f), std::vector<float>{1, 2, 3});
  CHECK(pa.params.weights.extent(0) == 2 && pa.params.bias.extent(0) == 3 && pa.get_num_trainable_parameters() == 9);
  // deep_copy and flatten
  View<float**, HostSpace> a("a", 2, 2);
  deep_copy(a, 1.5f);
  auto flat = flatten(a);
  static_assert(decltype(flat)::rank == 1);
  CHECK(flat.extent(0) == 4 && flat(3) == 1.5f && flat.data() == a.data());
}

// A view type of another library (as a Kokkos::View of device memory would
// be): data(), extent(), stride(), a LayoutRight layout and a device memory
// space.  The facade must copy it through the runtime, never read it on the host.
struct ForeignDeviceSpace {};
struct ForeignDeviceMatrix {
  using value_type = float;
  using array_layout = ponni::LayoutRight;
  using memory_space = ForeignDeviceSpace;
  static constexpr int rank = 2;
  float* p = nullptr;
  std::int64_t r = 0, c = 0, ld = 0;
  float* data() const { return p; }
  std::int64_t extent(int d) const { return d == 0 ? r : c; }
  std::int64_t stride(int d) const { return d == 0 ? ld : 1; }
};

template <class Model>
__global__ void in_kernel_sarray23(typename Model::Params p, float* result) {
  ponni::SArray<float, 2> in;
  ponni::SArray<float, 3> out;
  in(0) = 1.0f;
  in(1) = 2.0f;
  Model::forward_batch_parallel_in_kernel(in, out, p);
  for (int i = 0; i < 3; i++) result[i] = out(i);
}

void test_device_views_gpu() {
  using namespace ponni;
  using DeviceMatrix = View<float**, HIPSpace>;
  using DeviceVector = View<float*, HIPSpace>;
  {  // the README model (README.md:44-67), built from device Views
    DeviceMatrix weights_1("weights_1", 2, 3);
    DeviceVector bias_1("bias_1", 3);
    DeviceMatrix weights_2("weights_2", 3, 1);
    DeviceVector bias_2("bias_2", 1);
    deep_copy(weights_1, 0.25f);
    deep_copy(bias_1, 0.10f);
    deep_copy(weights_2, 0.50f);
    deep_copy(bias_2, -0.20f);
    auto model = create_inference_model(Matvec<float>(weights_1), Bias<float>(bias_1), Relu<float>(3),
                                        Matvec<float>(weights_2), Bias<float>(bias_2));
    model.validate();
    CHECK(model.get_layer<0>().params.weights.data() == weights_1.data());  // shared, not copied
    int const batch_size = 100000;
    DeviceMatrix inputs("inputs", 2, batch_size);
    deep_copy(inputs, 1.0f);
    auto outputs = model.forward_batch_parallel(inputs);
    auto const h = host(outputs);
    CHECK(near(h[0], 0.7, 1e-6) && near(h[batch_size - 1], 0.7, 1e-6));  // 3 x 0.5 x 0.6 - 0.2
    deep_copy(weights_1, 0.5f);  // a write through the shared View reaches the next pass
    auto const h2 = host(model.forward_batch_parallel(inputs));
    CHECK(near(h2[0], 1.45, 1e-6) && near(h2[batch_size / 2], 1.45, 1e-6));
  }
  {  // test_core_unit.cpp:516-546 with the weights shared
    DeviceMatrix mv_w("mv_w", 2, 3);
    mv_w.copy_from_host({1, 2, 3, 4, 5, 6});
    Matvec<float> mv(mv_w, true);
    CHECK(std::string(mv.get_label()) == "Matvec" && mv.get_num_trainable_parameters() == 6);
    CHECK(Matvec<float>::get_num_inputs(mv.params) == 2 && Matvec<float>::get_num_outputs(mv.params) == 3);
    DeviceVector mv_new_params("mv_new_params", 6);
    mv_new_params.copy_from_host({10, 11, 12, 13, 14, 15});
    mv.set_trainable_parameters(mv_new_params);
    auto got = host(mv.get_trainable_parameters());
    CHECK(near(got[0], 10.0, 0) && near(got[5], 15.0, 0));
    CHECK(host(mv_w)[0] == 10.0);  // the caller's View holds them
    auto m = create_inference_model(mv);
    auto y = host(m.forward_batch_parallel(device_matrix<float>(2, 1, {1, 2})));
    CHECK(y[0] == 36.0 && y[1] == 39.0 && y[2] == 42.0);
    using StaticMatvec = Matvec<float, 2, 3>;
    auto ms = create_inference_model(StaticMatvec(mv_w, true));
    View<float> r("r", 1, 3);
    using M = decltype(ms);
    hipLaunchKernelGGL((in_kernel_sarray23<M>), dim3(1), dim3(1), 0, 0, ms.params, r.data());
    CHECK(hipDeviceSynchronize() == hipSuccess);
    auto hr = host(r);
    CHECK(near(hr[0], 36.0, 1e-6) && near(hr[2], 42.0, 1e-6));
    mv_w.copy_from_host({1, 1, 1, 1, 1, 1});  // shared with `m` as well
    auto y1 = host(m.forward_batch_parallel(device_matrix<float>(2, 1, {1, 2})));
    CHECK(y1[0] == 3.0 && y1[2] == 3.0);
  }
  {  // host layers in a device model are copied (the rebind rule's other branch)
    View<float**, HostSpace> hw("hw", 2, 1);
    hw(0, 0) = 2.0f;
    hw(1, 0) = -1.0f;
    auto m = create_inference_model(Matvec<float, 1, 1, HostSpace>(hw));
    static_assert(std::is_same_v<std::decay_t<decltype(m.get_layer<0>())>, Matvec<float, 1, 1, HIPSpace>>);
    hw(0, 0) = 100.0f;  // not seen: the model holds a device copy
    auto y = host(m.forward_batch_parallel(device_matrix<float>(2, 1, {3, 1})));
    CHECK(y[0] == 5.0);
    // and a device layer in a host model (test_core_unit.cpp:380-404 spelling)
    auto hm = create_inference_model(DefaultHostExecutionSpace(), HostSpace(), Matvec<float>(ones(2, 2)),
                                     Bias<float>(std::vector<float>(2, 1.0f)), LeakyRelu<float>(2, 0.1f));
    View<float, HostSpace> hx("hx", 2, 1);
    hx(0, 0) = 1.0f;
    hx(1, 0) = 2.0f;
    auto hy = hm.forward_batch_parallel(hx);
    CHECK(near(hy(0, 0), 4.0, 1e-6) && near(hy(1, 0), 4.0, 1e-6));
  }
  {  // a foreign device view type: shared through its pointer, or copied by the runtime
    DeviceMatrix store("store", 2, 5);
    store.copy_from_host({10, 11, 12, 0, 0, 13, 14, 15, 0, 0});
    ForeignDeviceMatrix f{store.data(), 2, 3, 5};  // row stride 5
    Matvec<float> mv(f);
    CHECK(mv.params.weights.data() == store.data() && mv.params.weights.stride(0) == 5);
    auto m = create_inference_model(mv);
    auto y = host(m.forward_batch_parallel(device_matrix<float>(2, 1, {1, 2})));
    CHECK(y[0] == 36.0 && y[1] == 39.0 && y[2] == 42.0);
    Matvec<double> md(f);  // another element type: copied through the runtime
    CHECK((host(md.params.weights) == std::vector<double>{10, 11, 12, 13, 14, 15}));
    Bias<float> bf(ForeignDeviceMatrix{store.data(), 1, 3, 5});
    CHECK(bf.params.weights.data() == store.data() && bf.get_num_inputs() == 3);
  }
  {  // LayerNorm gamma / beta Views shared with the model
    DeviceVector g("g", 4), b("b", 4);
    deep_copy(g, 1.0f);
    auto m = create_inference_model(LayerNorm<float>(g, b));
    auto x = device_matrix<float>(4, 1, {1, 2, 3, 4});
    auto y0 = host(m.forward_batch_parallel(x));
    deep_copy(b, 2.0f);
    auto y1 = host(m.forward_batch_parallel(x));
    for (int i = 0; i < 4; i++) CHECK(near(y1[i] - y0[i], 2.0, 1e-5));
  }
}

}  // namespace

int main(int argc, char** argv) {
  bool const cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
  test_structure_and_planning<ponni::HostSpace>();
  test_parameters_and_fingerprint<ponni::HostSpace>();
  test_weights_files<ponni::HostSpace>();
  test_sixteen_bit_types();
  test_initializers_cpu();
  test_two_half_cpu();
  test_rebinding_cpu();
  test_user_layers_cpu();
  test_host_models_cpu();
  if (!cpu_only) {
    test_structure_and_planning<ponni::HIPSpace>();
    test_parameters_and_fingerprint<ponni::HIPSpace>();
    test_weights_files<ponni::HIPSpace>();
    test_device_views_gpu();
    test_user_layers_gpu();
    test_known_answers_gpu();
    test_views_streams_capacity_gpu();
    test_in_kernel_gpu();
    test_two_half_gpu();
  }
  std::printf("%s: %d checks, %d failures\n", cpu_only ? "cpu" : "cpu+gpu", g_checks, g_failures);
  return g_failures == 0 ? 0 : 1;
}
