// Generated-model headers (tests/cpp/gen/*.h, written by ponni_amd.emitter):
// C5Model (the c5 graph), TinyModel (a 3 -> 4 -> 2 graph) and F64Model (a
// double-precision narrow graph).  For the chosen model: load the weights file, run infer_batch
// (the header's ahead-of-time kernel), infer_batch_half2 and infer_one (an
// application kernel over device(); a kernel lambda that captures a copy of
// the model taken before load_weights, as the reference's test does; and on
// the host); then read the learned parameters, halve them through a device
// view, run infer_batch and every infer_one again and save the parameters.
// tests/test_cpp.py compares every output.  With --host (no GPU needed) only
// the host infer_one runs: y_host.bin, then y_host_scaled.bin after halving
// the parameters through set_parameters.
// Arrays on disk are raw Model::Scalar values (float, or double for F64Model).
//   test_generated <c5|tiny|f64> <weights.ponni> <x.bin [num_inputs, B]> <B> <out_dir> [--host]
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "gen/c5_model.h"
#include "gen/f64_model.h"
#include "gen/tiny_model.h"

template <class Model>
__global__ void infer_one_kernel(typename Model::Device m, typename Model::Scalar const* x, std::int64_t ldx,
                                 typename Model::Scalar* y, std::int64_t ldy, int batch) {
  int const b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  ponni::SArray<typename Model::Scalar, Model::num_inputs> in;
  ponni::SArray<typename Model::Scalar, Model::num_outputs> out;
  for (int f = 0; f < Model::num_inputs; f++) in(f) = x[f * ldx + b];
  m.infer_one(in, out);
  for (int f = 0; f < Model::num_outputs; f++) y[f * ldy + b] = out(f);
}

template <class F>
__global__ void for_each_sample(int batch, F f) {
  int const b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < batch) f(b);
}

template <class T>
static std::vector<T> read_raw(char const* path, std::size_t n) {
  std::vector<T> v(n);
  FILE* f = std::fopen(path, "rb");
  if (!f || std::fread(v.data(), sizeof(T), n, f) != n) ponni::abort(std::string("cannot read ") + path);
  std::fclose(f);
  return v;
}

template <class T>
static void write_raw(std::string const& path, std::vector<T> const& v) {
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f || std::fwrite(v.data(), sizeof(T), v.size(), f) != v.size()) ponni::abort("cannot write " + path);
  std::fclose(f);
}

// infer_one on the host, sample by sample, for x [num_inputs, B] (row stride B).
template <class Model>
std::vector<typename Model::Scalar> host_outputs(Model const& m, std::vector<typename Model::Scalar> const& x,
                                                 int B) {
  using T = typename Model::Scalar;
  std::vector<T> out(std::size_t(Model::num_outputs) * B);
  for (int b = 0; b < B; b++) {
    ponni::SArray<T, Model::num_inputs> in;
    ponni::SArray<T, Model::num_outputs> o;
    for (int f = 0; f < Model::num_inputs; f++) in(f) = x[std::size_t(f) * B + b];
    m.infer_one(in, o);
    for (int f = 0; f < Model::num_outputs; f++) out[std::size_t(f) * B + b] = o(f);
  }
  return out;
}

template <class Model>
int run_host(char const* weights, char const* xpath, int B, std::string const& dir) {
  using T = typename Model::Scalar;
  Model m;
  Model const early = m;  // sees the weights loaded below
  std::string err;
  if (!m.load_weights(weights, &err)) {
    std::fprintf(stderr, "load_weights: %s\n", err.c_str());
    return 1;
  }
  std::vector<T> const xh = read_raw<T>(xpath, std::size_t(Model::num_inputs) * B);
  write_raw(dir + "/y_host.bin", host_outputs(early, xh, B));
  std::vector<T> p(Model::get_num_parameters());
  m.get_parameters(p);
  for (T& v : p) v *= T(0.5);
  m.set_parameters(p);
  write_raw(dir + "/y_host_scaled.bin", host_outputs(early, xh, B));
  std::printf("test_generated --host: wrote %d samples (%s)\n", B, Model::model_fingerprint().c_str());
  return 0;
}

template <class Model>
int run(char const* weights, char const* xpath, int B, std::string const& dir) {
  using T = typename Model::Scalar;
  Model m;
  // A copy taken now shares what load_weights and set_parameters change later
  // (src/generator/tests/test_generated.cpp:174-184 copies after loading).
  Model const early = m;
  std::string err;
  if (m.weights_loaded() || m.parameters_are_finite() || m.save_parameters(dir + "/early.ponni", &err)) {
    std::fprintf(stderr, "a model without weights must report them missing\n");
    return 1;
  }
  if (m.load_weights(dir + "/missing.ponni", &err) || err.empty()) {
    std::fprintf(stderr, "loading a missing file must fail with a message\n");
    return 1;
  }
  if (!m.load_weights(weights, &err)) {
    std::fprintf(stderr, "load_weights: %s\n", err.c_str());
    return 1;
  }
  std::vector<T> const xh = read_raw<T>(xpath, std::size_t(Model::num_inputs) * B);
  ponni::View<T> x("x", Model::num_inputs, B);
  x.copy_from_host(xh);
  ponni::View<T> y("y", Model::num_outputs, B), yh("yh", Model::num_outputs, B), y1("y1", Model::num_outputs, B),
      yc("yc", Model::num_outputs, B);
  auto one = [&] {
    hipLaunchKernelGGL(infer_one_kernel<Model>, dim3((B + 127) / 128), dim3(128), 0, 0, m.device(), x.data(),
                       x.stride(0), y1.data(), y1.stride(0), B);
    return hipDeviceSynchronize() == hipSuccess;
  };
  // The model itself captured by value in an application kernel.
  auto captured = [&] {
    T const* xp = x.data();
    T* yp = yc.data();
    std::int64_t const ldx = x.stride(0), ldy = yc.stride(0);
    Model const model = early;
    auto body = [=] __device__(int b) {
      ponni::SArray<T, Model::num_inputs> in;
      ponni::SArray<T, Model::num_outputs> out;
      for (int f = 0; f < Model::num_inputs; f++) in(f) = xp[f * ldx + b];
      model.infer_one(in, out);
      for (int f = 0; f < Model::num_outputs; f++) yp[f * ldy + b] = out(f);
    };
    hipLaunchKernelGGL(for_each_sample<decltype(body)>, dim3((B + 127) / 128), dim3(128), 0, 0, B, body);
    return hipDeviceSynchronize() == hipSuccess;
  };
  auto host = [&] { return host_outputs(early, xh, B); };
  m.infer_batch(x, y);
  m.infer_batch_half2(x, yh);
  if (!one() || !captured()) return 1;
  write_raw(dir + "/y_batch.bin", y.copy_to_host());
  write_raw(dir + "/y_half.bin", yh.copy_to_host());
  write_raw(dir + "/y_one.bin", y1.copy_to_host());
  write_raw(dir + "/y_copy.bin", yc.copy_to_host());
  write_raw(dir + "/y_host.bin", host());
  if (!m.weights_loaded() || !m.parameters_are_finite() || !m.parameters_synchronized()) return 1;

  std::vector<T> p(Model::get_num_parameters());
  m.get_parameters(p);
  write_raw(dir + "/params.bin", p);
  for (T& v : p) v *= T(0.5);
  ponni::View<T> pv("p", 1, Model::get_num_parameters());
  pv.copy_from_host(p);
  m.set_parameters(pv);
  m.infer_batch(x, y);
  if (!one() || !captured()) return 1;
  write_raw(dir + "/y_batch_scaled.bin", y.copy_to_host());
  write_raw(dir + "/y_one_scaled.bin", y1.copy_to_host());
  write_raw(dir + "/y_copy_scaled.bin", yc.copy_to_host());
  write_raw(dir + "/y_host_scaled.bin", host());
  if (!m.save_parameters(dir + "/saved.ponni", &err)) {
    std::fprintf(stderr, "save_parameters: %s\n", err.c_str());
    return 1;
  }
  std::printf("test_generated: wrote %d samples (%s)\n", B, Model::model_fingerprint().c_str());
  return 0;
}

int main(int argc, char** argv) {
  bool const host = argc == 7 && std::strcmp(argv[6], "--host") == 0;
  if (argc != 6 && !host) {
    std::fprintf(stderr, "usage: %s c5|tiny|f64 weights.ponni x.bin batch out_dir [--host]\n", argv[0]);
    return 2;
  }
  int const B = std::atoi(argv[4]);
  using namespace ponni::generated;
  if (std::strcmp(argv[1], "c5") == 0)
    return host ? run_host<C5Model>(argv[2], argv[3], B, argv[5]) : run<C5Model>(argv[2], argv[3], B, argv[5]);
  if (std::strcmp(argv[1], "tiny") == 0)
    return host ? run_host<TinyModel>(argv[2], argv[3], B, argv[5]) : run<TinyModel>(argv[2], argv[3], B, argv[5]);
  if (std::strcmp(argv[1], "f64") == 0)
    return host ? run_host<F64Model>(argv[2], argv[3], B, argv[5]) : run<F64Model>(argv[2], argv[3], B, argv[5]);
  std::fprintf(stderr, "unknown model %s\n", argv[1]);
  return 2;
}
