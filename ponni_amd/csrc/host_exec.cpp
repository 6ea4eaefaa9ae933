// Host execution-space models: the plan's GENERIC op list evaluated on the
// host, one sample at a time, by the same per-sample interpreter the GENERIC
// kernel and the in-kernel API run (generic_ops.h).  The reference gets this
// by instantiating its Inference on a host execution space
// (create_inference_model(DefaultHostExecutionSpace(), HostSpace(), ...),
// tests/unit/test_core_unit.cpp:380-404); here the caller asks for it
// explicitly through ponni_forward_host -- nothing on the device path ever
// lands here.
#include <algorithm>
#include <cstring>
#include <system_error>
#include <thread>
#include <vector>

#include "generic_ops.h"
#include "plan.h"

using namespace ponni_hip;

namespace {

// Samples [b0, b1) with thread-private states (feature-contiguous, ld = 1).
template <class real>
void run_range(ponni_plan_s const& t, real const* params, real const* x, int64_t ldx, real* y, int64_t ldy,
               int64_t b0, int64_t b1) {
  int const width = std::max({t.max_width, t.tmp_features[0], t.tmp_features[1], 1});
  std::vector<real> tmp1(width), tmp2(width), saved(std::max(t.saved_total, 1));
  Bufs buf;
  buf.fixed[BUF_TMP1] = {reinterpret_cast<char*>(tmp1.data()), 1};
  buf.fixed[BUF_TMP2] = {reinterpret_cast<char*>(tmp2.data()), 1};
  buf.saved = {reinterpret_cast<char*>(saved.data()), 1};
  buf.slot_row = t.slot_rows.data();
  int const num_ops = static_cast<int>(t.ops.size());
  for (int64_t b = b0; b < b1; b++) {
    buf.fixed[BUF_INPUT] = {reinterpret_cast<char*>(const_cast<real*>(x + b)), ldx};
    buf.fixed[BUF_OUTPUT] = {reinterpret_cast<char*>(y + b), ldy};
    run_ops<real>(t.ops.data(), num_ops, t.steps.data(), params, buf, 0);
  }
}

template <class real>
void run_all(ponni_plan_s const& t, real const* params, void const* x, int64_t ldx, void* y, int64_t ldy,
             int64_t batch, int threads) {
  auto const* xr = static_cast<real const*>(x);
  auto* yr = static_cast<real*>(y);
  // At least 256 samples per thread: thread start-up is not free.
  int64_t const n = std::max<int64_t>(1, std::min<int64_t>(threads, (batch + 255) / 256));
  if (n == 1) {
    run_range<real>(t, params, xr, ldx, yr, ldy, 0, batch);
    return;
  }
  std::vector<std::thread> pool;
  pool.reserve(static_cast<size_t>(n));
  int64_t done = n;  // slices from here on run on the calling thread
  for (int64_t i = 0; i < n; i++) {
    int64_t const b0 = batch * i / n, b1 = batch * (i + 1) / n;
    try {
      pool.emplace_back([&, b0, b1] { run_range<real>(t, params, xr, ldx, yr, ldy, b0, b1); });
    } catch (std::system_error const&) {  // no more threads: finish here
      done = i;
      break;
    }
  }
  if (done < n) run_range<real>(t, params, xr, ldx, yr, ldy, batch * done / n, batch);
  for (auto& th : pool) th.join();
}

int check_host_plan(ponni_plan plan) {
  if (plan == nullptr) return set_error(PONNI_ERR_INVALID_ARGUMENT, "plan is null");
  if (plan->dtype != PONNI_F32 && plan->dtype != PONNI_F64)
    return set_error(PONNI_ERR_UNSUPPORTED, "host execution runs F32 and F64 models");
  return PONNI_OK;
}

}  // namespace

extern "C" {

int ponni_plan_host_model(ponni_plan plan, ponni_device_model* out) {
  int st = check_host_plan(plan);
  if (st != PONNI_OK) return st;
  if (out == nullptr) return set_error(PONNI_ERR_INVALID_ARGUMENT, "output is null");
  ponni_plan_s* t = nullptr;
  st = host_twin(*plan, t);
  if (st != PONNI_OK) return st;
  std::memset(out, 0, sizeof(*out));
  out->ops = t->ops.data();
  out->steps = t->steps.data();
  out->params = t->dtype == PONNI_F64 ? static_cast<void const*>(t->host_params_f64.data())
                                      : static_cast<void const*>(t->host_params_f32.data());
  out->num_ops = static_cast<int32_t>(t->ops.size());
  out->dtype = t->dtype;
  out->num_inputs = t->layers.front().n_in;
  out->num_outputs = t->layers.back().n_out;
  out->max_width = t->max_width;
  out->tmp_features[0] = t->tmp_features[0];
  out->tmp_features[1] = t->tmp_features[1];
  out->num_slots = t->num_slots;
  out->saved_total = t->saved_total;
  out->slot_rows = t->slot_rows.data();
  return PONNI_OK;
}

int ponni_forward_host(ponni_plan plan, const void* x, int64_t ld_in, void* y, int64_t ld_out, int64_t batch,
                       int32_t threads) {
  int st = check_host_plan(plan);
  if (st != PONNI_OK) return st;
  if (plan->external)
    return set_error(PONNI_ERR_UNSUPPORTED,
                     "the plan holds external (custom) layers: run it through ponni_plan_host_model");
  if (batch <= 0) return set_error(PONNI_ERR_SHAPE, "Inference requires a nonzero batch size");
  if (batch > INT32_MAX) return set_error(PONNI_ERR_SHAPE, "batch exceeds INT_MAX");
  if (x == nullptr || y == nullptr) return set_error(PONNI_ERR_INVALID_ARGUMENT, "input or output pointer is null");
  if (ld_in < batch || ld_out < batch)
    return set_error(PONNI_ERR_SHAPE, "Error: Provided output dimensions do not match the model and input batch");
  if (threads < 0) return set_error(PONNI_ERR_INVALID_ARGUMENT, "thread count must be nonnegative");
  ponni_plan_s* t = nullptr;
  st = host_twin(*plan, t);
  if (st != PONNI_OK) return st;
  int const n = threads > 0 ? threads : std::max(1u, std::thread::hardware_concurrency());
  if (t->dtype == PONNI_F64) run_all<double>(*t, t->host_params_f64.data(), x, ld_in, y, ld_out, batch, n);
  else run_all<float>(*t, t->host_params_f32.data(), x, ld_in, y, ld_out, batch, n);
  return PONNI_OK;
}

}  // extern "C"
