// Framework integration tests restated against the facade: a model exported
// from PyTorch into a .ponni file (weights plus test.input / test.output,
// written by tests/test_frameworks.py) is rebuilt in template mode from the
// file's tensors and must reproduce the framework's outputs within 1e-5, as
// unit/pytorch_resnet/test_pytorch_resnet.cpp:20-77 and
// unit/projection_skip/test_projection_skip.cpp:20-53 do.
//   test_frameworks <resnet|projection> <file.ponni> [--host]
// --host runs the model on the host execution space (no GPU needed).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>

#include "ponni.h"

namespace {

// Layers live in the model's memory space, so the host run needs no device.
template <class Space, class Exec>
auto resnet(ponni::PonniFile const& f, Exec const& exec) {
  using namespace ponni;
  using Mv = Matvec<float, 1, 1, Space>;
  using B = Bias<float, 1, Space>;
  using Act = Silu<float, 1, Space>;
  using Save = Save_State<0, float, 1, Space>;
  using Add = Binop_Add<0, float, 1, Space>;
  auto w = [&](char const* name) { return load_ponni_tensor<2, Space>(f, name); };
  auto v = [&](char const* name) { return load_ponni_tensor<1, Space>(f, name); };
  return create_inference_model(exec, Space(), Mv(w("fc1.weight")), B(v("fc1.bias")), Act(5), Save(5),
                                Mv(w("fc2.weight")), B(v("fc2.bias")), Act(5), Add(5), Save(5), Mv(w("fc3.weight")),
                                B(v("fc3.bias")), Act(5), Add(5), Save(5), Mv(w("fc4.weight")), B(v("fc4.bias")),
                                Act(5), Add(5), Mv(w("fc5.weight")), B(v("fc5.bias")));
}

template <class Space, class Exec>
auto projection(ponni::PonniFile const& f, Exec const& exec) {
  using namespace ponni;
  auto w_main = load_ponni_tensor<2, Space>(f, "w_main");
  auto b_main = load_ponni_tensor<1, Space>(f, "b_main");
  auto w_skip = load_ponni_tensor<2, Space>(f, "w_skip");
  auto b_skip = load_ponni_tensor<1, Space>(f, "b_skip");
  return create_inference_model(exec, Space(), Relu<float, 1, Space>(2), Save_State<0, float, 1, Space>(2),
                                Matvec<float, 1, 1, Space>(w_main, false), Bias<float, 1, Space>(b_main, false),
                                Binop_Projection_Add<0, float, 3, 2, Space>(w_skip, b_skip, false));
}

template <class Space, class Model>
int check(Model& model, ponni::PonniFile const& f) {
  model.validate();
  auto in = ponni::load_ponni_tensor<2, Space>(f, "test.input");
  auto expected = ponni::create_host_copy(ponni::load_ponni_tensor<2, Space>(f, "test.output"));
  auto out = ponni::create_host_copy(model.forward_batch_parallel(in));
  if (out.extent(0) != expected.extent(0) || out.extent(1) != expected.extent(1)) {
    std::fprintf(stderr, "output shape mismatch\n");
    return 1;
  }
  double worst = 0;
  for (std::int64_t j = 0; j < out.extent(1); j++)
    for (std::int64_t i = 0; i < out.extent(0); i++) worst = std::fmax(worst, std::fabs(out(i, j) - expected(i, j)));
  std::printf("max |difference| %.3g over %lld samples\n", worst, static_cast<long long>(out.extent(1)));
  return worst <= 1e-5 ? 0 : 1;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 3) {
    std::fprintf(stderr, "usage: %s resnet|projection file.ponni [--host]\n", argv[0]);
    return 2;
  }
  bool const host = argc > 3 && std::strcmp(argv[3], "--host") == 0;
  ponni::PonniFile f;
  std::string error;
  if (!f.load(argv[2], &error)) {
    std::fprintf(stderr, "%s\n", error.c_str());
    return 1;
  }
  bool const res = std::strcmp(argv[1], "resnet") == 0;
  if (host) {
    if (res) {
      auto m = resnet<ponni::HostSpace>(f, ponni::Host());
      return check<ponni::HostSpace>(m, f);
    }
    auto m = projection<ponni::HostSpace>(f, ponni::Host());
    return check<ponni::HostSpace>(m, f);
  }
  if (res) {
    auto m = resnet<ponni::HIPSpace>(f, ponni::HIP());
    return check<ponni::HIPSpace>(m, f);
  }
  auto m = projection<ponni::HIPSpace>(f, ponni::HIP());
  return check<ponni::HIPSpace>(m, f);
}
