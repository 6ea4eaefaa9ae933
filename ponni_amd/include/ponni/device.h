// ponni/device.h -- per-sample inference inside application kernels (HIP).
//
// The reference lets code that already runs inside a Kokkos kernel evaluate
// one sample of a model: Inference::forward_batch_parallel_in_kernel, in a
// View form (sample `ibatch` of [features, batch] LayoutRight views,
// src/ponni_Inference.h:394-408) and an SArray form (fixed-size per-thread
// arrays, :592-665), both given the model's `params`.  Here the model's
// device description comes from ponni_plan_device_model (include/ponni_hip.h):
// the plan's GENERIC op list and parameters in device memory.  forward_one
// walks that op list for one sample -- the same per-sample interpreter the
// GENERIC batch kernel runs (csrc/generic_ops.h) -- with the intermediate
// states (tmp1, tmp2, saved slots) in the calling thread's private memory
// rather than in [width, capacity] HBM scratch.
//
// Build: hipcc ... -I<repo>/include -I<repo>/ponni_amd/include
#pragma once

#include <hip/hip_runtime.h>

#include "../../../include/ponni_hip.h"
#include "../../csrc/generic_ops.h"

namespace ponni {

// Thread-private state limits of forward_one: the widest state of the chain
// (MAXW features) and all saved slots together (MAXSAVED features, any
// number of slots).
constexpr int kInKernelMaxWidth = 256;
constexpr int kInKernelMaxSaved = 512;

// Can forward_one<real, MAXW, MAXSAVED> evaluate this model?
template <int MAXW = kInKernelMaxWidth, int MAXSAVED = kInKernelMaxSaved>
__host__ __device__ inline bool fits_in_kernel(ponni_device_model const& m) {
  return m.max_width <= MAXW && m.tmp_features[0] <= MAXW && m.tmp_features[1] <= MAXW && m.saved_total <= MAXSAVED;
}

// One sample: out[f * out_ld] = model(in[k * in_ld]) for f < num_outputs.
// Device code passes the description ponni_plan_device_model gives; host
// code (host execution-space models) the one ponni_plan_host_model gives.
// `real` is float for F32 models and double for F64 models.  A model that
// does not fit the thread-private limits, or of another dtype, writes NaN.
// `ext` evaluates the chain's caller-implemented layers (PONNI_LAYER_EXTERNAL),
// see ponni_hip::run_ops; the facade supplies it for user layer types.
template <class real, int MAXW = kInKernelMaxWidth, int MAXSAVED = kInKernelMaxSaved,
          class Ext = ponni_hip::NoExternal>
__host__ __device__ inline void forward_one(ponni_device_model const& m, real const* in, int64_t in_ld, real* out,
                                   int64_t out_ld, Ext const& ext = Ext()) {
  constexpr int want = sizeof(real) == 8 ? PONNI_F64 : PONNI_F32;
  if (m.dtype != want || !fits_in_kernel<MAXW, MAXSAVED>(m)) {
    for (int f = 0; f < m.num_outputs; f++) out[f * out_ld] = real(__builtin_nan(""));
    return;
  }
  real tmp[2][MAXW];
  real saved[MAXSAVED];
  ponni_hip::Bufs buf;
  buf.fixed[ponni_hip::BUF_INPUT] = {reinterpret_cast<char*>(const_cast<real*>(in)), in_ld};
  buf.fixed[ponni_hip::BUF_OUTPUT] = {reinterpret_cast<char*>(out), out_ld};
  buf.fixed[ponni_hip::BUF_TMP1] = {reinterpret_cast<char*>(tmp[0]), 1};
  buf.fixed[ponni_hip::BUF_TMP2] = {reinterpret_cast<char*>(tmp[1]), 1};
  buf.saved = {reinterpret_cast<char*>(saved), 1};
  buf.slot_row = m.slot_rows;
  ponni_hip::run_ops<real>(static_cast<ponni_hip::Op const*>(m.ops), m.num_ops,
                           static_cast<ponni_hip::Step const*>(m.steps), static_cast<real const*>(m.params), buf,
                           0, ext);
}

// One sample through a program fixed at compile time: Program holds the
// plan's GENERIC op list as constexpr members (the text
// ponni_plan_program_source writes, which generated model headers embed),
// so every op is expanded in place with its sizes and offsets as constants
// and the thread-private states are sized to the plan (the reference
// emitter's per-model infer_one body with planned local storage,
// kokkos_nn/emitter.py:1897-1901).  params: the parameters of the same
// plan's ponni_plan_device_model (device code) or ponni_plan_host_model
// (host code) description; Program::dtype must match `real`.
template <class real, class Program, class Ext = ponni_hip::NoExternal>
__host__ __device__ inline void forward_one_program(void const* params, real const* in, int64_t in_ld, real* out,
                                                    int64_t out_ld, Ext const& ext = Ext()) {
  static_assert(Program::dtype == (sizeof(real) == 8 ? PONNI_F64 : PONNI_F32), "program dtype and real differ");
  constexpr int t1 = Program::tmp_features[0] > 0 ? Program::tmp_features[0] : 1;
  constexpr int t2 = Program::tmp_features[1] > 0 ? Program::tmp_features[1] : 1;
  constexpr int sv = Program::saved_total > 0 ? Program::saved_total : 1;
  real tmp1[t1], tmp2[t2], saved[sv];
  ponni_hip::Bufs buf;
  buf.fixed[ponni_hip::BUF_INPUT] = {reinterpret_cast<char*>(const_cast<real*>(in)), in_ld};
  buf.fixed[ponni_hip::BUF_OUTPUT] = {reinterpret_cast<char*>(out), out_ld};
  buf.fixed[ponni_hip::BUF_TMP1] = {reinterpret_cast<char*>(tmp1), 1};
  buf.fixed[ponni_hip::BUF_TMP2] = {reinterpret_cast<char*>(tmp2), 1};
  buf.saved = {reinterpret_cast<char*>(saved), 1};
  buf.slot_row = Program::slot_rows;
  ponni_hip::run_program<real, Program, Ext>(static_cast<real const*>(params), buf, 0, ext,
                                             std::make_integer_sequence<int, Program::num_ops>());
}

}  // namespace ponni
