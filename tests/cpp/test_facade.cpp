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

auto four_block_model() {
  using namespace ponni;
  return create_inference_model(
      Matvec<float>(ones(2, 5)), Bias<float>(std::vector<float>(5, 0.5f)), Relu<float>(5), Tanh<float>(5),
      Matvec<float>(ones(5, 3)), Bias<float>(std::vector<float>(3, -0.25f)), Sigmoid<float>(3),
      Matvec<float>(ones(3, 7)), Bias<float>(std::vector<float>(7, 0.1f)), LeakyRelu<float>(7, 0.2f),
      Matvec<float>(ones(7, 2)), Bias<float>(std::vector<float>(2, -0.2f)), HardSwish<float>(2));
}

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

void test_structure_and_planning() {
  using namespace ponni;
  auto first = create_inference_model(Matvec<float>(ones(2, 2)), Bias<float>(std::vector<float>{1, 1}),
                                      LeakyRelu<float>(2, 0.1f));
  CHECK(first.get_num_inputs() == 2 && first.get_num_outputs() == 2);
  CHECK(first.get_planned_temporary_size<0>() == 0 && first.get_planned_temporary_size<1>() == 0);
  CHECK(first.get_num_fused_dense_blocks() == 1);
  auto four = four_block_model();
  CHECK(four.get_planned_temporary_size<0>() == 7 && four.get_planned_temporary_size<1>() == 3);
  CHECK(four.get_num_fused_dense_blocks() == 4);
  four.validate();
  auto soft = create_inference_model(Matvec<float>(ones(2, 3)), Bias<float>(std::vector<float>{0, 1, 2}),
                                     Relu<float>(3), Softmax<float>(3), Matvec<float>(ones(3, 2)),
                                     Bias<float>(std::vector<float>{0, -1}), Tanh<float>(2));
  CHECK(soft.get_planned_temporary_size<0>() == 3 && soft.get_planned_temporary_size<1>() == 0);
  auto res = create_inference_model(Save_State<0>(2), Relu<float>(2), Binop_Concatenate<0>(2, 4, true),
                                    Save_State<1>(4), Relu<float>(4), Binop_Add<1>(4),
                                    Binop_Concatenate<0>(4, 6, true));
  CHECK(res.get_num_saved_states() == 2);
  res.validate();
}

void test_parameters_and_fingerprint() {
  using namespace ponni;
  ponni::Matrix<float> w(2, 3, std::vector<float>{1, 2, 3, 4, 5, 6});
  auto m = create_inference_model(Matvec<float>(w), Bias<float>(std::vector<float>{7, 8, 9}), Relu<float>(3),
                                  LayerNorm<float>(3), Matvec<float>(ones(3, 1), false));
  CHECK(m.get_num_trainable_parameters() == 6 + 3 + 6);  // the last Matvec is frozen
  auto p = m.get_trainable_parameters();
  std::vector<float> want{1, 2, 3, 4, 5, 6, 7, 8, 9, 1, 1, 1, 0, 0, 0};
  CHECK(p.size() == want.size() && std::equal(p.begin(), p.end(), want.begin()));
  std::vector<float> q(15);
  for (int i = 0; i < 15; i++) q[i] = 0.5f * i;
  m.set_trainable_parameters(q);
  p = m.get_trainable_parameters();
  CHECK(std::equal(p.begin(), p.end(), q.begin()));
  CHECK(m.get_layer<1>().params[0] == 3.0);
  // "ponni-template-model-v1\n" + "I\tlabel\tnin\tnout\tntrainable\n" (ponni_Inference.h:270-288)
  std::string text = "ponni-template-model-v1\n0\tMatvec\t2\t3\t6\n1\tBias\t3\t3\t3\n2\tReLU\t3\t3\t0\n"
                     "3\tLayerNorm\t3\t3\t6\n4\tMatvec\t3\t1\t0\n";
  std::string fp = ponni::ponni_fnv1a64_string(
      ponni::ponni_fnv1a64(reinterpret_cast<unsigned char const*>(text.data()), text.size()));
  CHECK(m.weight_schema_fingerprint() == fp);
}

void test_weights_files() {
  using namespace ponni;
  char const* path = "/tmp/ponni_facade_test.ponni";
  auto a = create_inference_model(Matvec<float>(ponni::Matrix<float>(2, 2, std::vector<float>{1, 2, 3, 4})),
                                  Bias<float>(std::vector<float>{5, 6}));
  std::string err;
  CHECK(a.save_weights(path, &err));
  auto b = create_inference_model(Matvec<float>(ones(2, 2)), Bias<float>(std::vector<float>{0, 0}));
  CHECK(b.load_weights(path, &err));
  auto p = b.get_trainable_parameters();
  CHECK(p.size() == 6 && p[0] == 1 && p[3] == 4 && p[5] == 6);
  auto c = create_inference_model(Matvec<float>(ones(2, 2)), Relu<float>(2), Bias<float>(std::vector<float>{0, 0}));
  CHECK(!c.load_weights(path, &err));
  CHECK(err.find("fingerprint") != std::string::npos);
  auto d = create_inference_model(Relu<float>(2));
  CHECK(!d.load_weights(path, &err));
  CHECK(err == "cannot load weights into a model with no trainable parameters");
  CHECK(!d.save_weights(path, &err));
  CHECK(err == "cannot save weights from a model with no trainable parameters");
  auto e = create_inference_model_double_precision(Matvec<double>(ones(2, 2)), Bias<double>(std::vector<double>{0, 0}));
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
  // Parameter edits through get_layer + mark_modified reach the device.
  auto one = create_inference_model(Matvec<float>(ones(2, 1)));
  one.get_layer<0>().params = {3.0, 4.0};
  one.get_layer<0>().mark_modified();
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
template <class Exec>
auto four_block_model_on(Exec const& exec) {
  using namespace ponni;
  return create_inference_model(
      exec, Matvec<float>(ones(2, 5)), Bias<float>(std::vector<float>(5, 0.5f)), Relu<float>(5), Tanh<float>(5),
      Matvec<float>(ones(5, 3)), Bias<float>(std::vector<float>(3, -0.25f)), Sigmoid<float>(3),
      Matvec<float>(ones(3, 7)), Bias<float>(std::vector<float>(7, 0.1f)), LeakyRelu<float>(7, 0.2f),
      Matvec<float>(ones(7, 2)), Bias<float>(std::vector<float>(2, -0.2f)), HardSwish<float>(2));
}

void test_host_models_cpu() {
  using namespace ponni;
  {  // test_core_unit.cpp:380-404
    auto host_model = create_inference_model(DefaultHostExecutionSpace(), HostSpace(), Matvec<float>(ones(2, 2)),
                                             Bias<float>(std::vector<float>(2, 1.0f)), LeakyRelu<float>(2, 0.1f));
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
    auto m = four_block_model_on(Host(3));
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
    auto mixed = create_inference_model(Host(), HostSpace(), Matvec<float>(w),
                                        Bias<float>(std::vector<float>{0.1f, -0.2f}), TestIndexedPointwise<float, 2>(),
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
    auto m = detail::create_model<double>(Host(), HostSpace(), Matvec<double>(Matrix<double>(3, 2, 1.0)),
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
    auto p = m.get_trainable_parameters();
    for (auto& v : p) v *= 2.0f;
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

}  // namespace

int main(int argc, char** argv) {
  bool const cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
  test_structure_and_planning();
  test_parameters_and_fingerprint();
  test_weights_files();
  test_sixteen_bit_types();
  test_user_layers_cpu();
  test_host_models_cpu();
  if (!cpu_only) {
    test_user_layers_gpu();
    test_known_answers_gpu();
    test_views_streams_capacity_gpu();
    test_in_kernel_gpu();
  }
  std::printf("%s: %d checks, %d failures\n", cpu_only ? "cpu" : "cpu+gpu", g_checks, g_failures);
  return g_failures == 0 ? 0 : 1;
}
