// One sample's pass through a lowered op list (program.h), reading and
// writing states through View2 handles: element (f, b) of a handle is
// base[f * ld + b].  The GENERIC kernel runs it per lane over the plan's HBM
// scratch (b = the lane's sample); the in-kernel per-sample API
// (ponni/device.h) runs it over thread-private arrays (ld = 1, b = 0), in
// device code and, for host execution-space models, on the host.
// Each case follows the reference layer it cites.
#pragma once

#include <utility>

#include "../../include/ponni_hip.h"
#include "pointwise.h"
#include "program.h"

namespace ponni_hip {

// F16 / BF16 storage computes in fp32; load_as / store_as are specialized for
// those storage types where they are used (kernels_generic.hip).
template <class S> struct Compute { using type = float; };
template <> struct Compute<double> { using type = double; };

template <class S> __host__ __device__ inline typename Compute<S>::type load_as(S const* p) {
  return static_cast<typename Compute<S>::type>(*p);
}

template <class S, class C> __host__ __device__ inline void store_as(S* p, C v) { *p = static_cast<S>(v); }

struct View2 {
  char* base;
  int64_t ld;
};

template <class S>
__host__ __device__ inline S* at(View2 const& v, int f, int64_t b) {
  return reinterpret_cast<S*>(v.base) + (int64_t(f) * v.ld + b);
}

// The state handles of one sample's pass: input, output, tmp1 and tmp2
// (fixed[Buffer]), and the saved slots, which share one area of the same
// row stride -- slot s holds rows slot_row[s] .. slot_row[s] +
// get_saved_state_size<s>() - 1 of `saved` -- so a plan may use any number
// of slots.  slot_row has at least one entry (0 for a plan with no slot).
struct Bufs {
  View2 fixed[BUF_SAVED];
  View2 saved;
  int32_t const* slot_row;
};

template <class S>
__host__ __device__ inline View2 slot_view(Bufs const& B, int s) {
  return View2{reinterpret_cast<char*>(reinterpret_cast<S*>(B.saved.base) + int64_t(B.slot_row[s]) * B.saved.ld),
               B.saved.ld};
}

template <class S>
__host__ __device__ inline View2 buf_view(Bufs const& B, int id) {
  return id < BUF_SAVED ? B.fixed[id] : slot_view<S>(B, id - BUF_SAVED);
}

// Caller-implemented layers (OP_EXTERNAL) are evaluated by `ext`:
// ext(index, flags, in, out, saved, n_in, n_out, b) with the state handles of
// the op; the library's own kernels never see such an op.
struct NoExternal {
  __host__ __device__ void operator()(int, int, View2 const&, View2 const&, View2 const&, int, int, int64_t) const {}
};

// One op of a plan's program for sample b.  Inlined into its caller, so a
// caller that passes an op known at compile time (run_program) gets the op's
// branch alone, with its sizes and offsets as constants.
template <class S, class Ext = NoExternal>
__host__ __device__ __attribute__((always_inline)) inline void run_op(
    Op const op, Step const* __restrict__ steps, typename Compute<S>::type const* __restrict__ params,
    Bufs const& buf, int64_t b, Ext const& ext) {
  using C = typename Compute<S>::type;
  {
    View2 const in = buf_view<S>(buf, op.src);
    View2 const out = buf_view<S>(buf, op.dst);
    switch (op.code) {
      case OP_DENSE: {
        // ponni_Inference.h:431-444 with Matvec::compute_output (ponni_Matvec.h:70-79).
        // A generated Dense seeds the sum with its bias (emitter.py:701-710).
        C const* w = params + op.woff;
        int const first = (op.aux & DENSE_BIAS_FIRST) ? 1 : 0;
        for (int f = 0; f < op.n_out; f++) {
          C v = first ? params[steps[op.epi_begin].off + f] : C(0);
          for (int k = 0; k < op.n_in; k++) v += w[int64_t(k) * op.n_out + f] * load_as<S>(at<S>(in, k, b));
          for (int s = first; s < op.epi_count; s++) {
            Step const st = steps[op.epi_begin + s];
            C const bias = act_has_param(st.act) ? params[st.off + f] : C(0);
            v = apply_step<C>(st.act, v, bias, C(st.a), C(st.b));
          }
          store_as<S, C>(at<S>(out, f, b), v);
        }
        break;
      }
      case OP_POINTWISE: {
        Step const st = steps[op.epi_begin];
        for (int f = 0; f < op.n_out; f++) {
          C const bias = act_has_param(st.act) ? params[st.off + f] : C(0);
          store_as<S, C>(at<S>(out, f, b), apply_step<C>(st.act, load_as<S>(at<S>(in, f, b)), bias, C(st.a), C(st.b)));
        }
        break;
      }
      case OP_LAYER_NORM: {  // ponni_LayerNorm.h:76-99
        int const n = op.n_in;
        C mean = C(0);
        for (int f = 0; f < n; f++) mean += load_as<S>(at<S>(in, f, b));
        mean /= C(n);
        C var = C(0);
        for (int f = 0; f < n; f++) {
          C const d = load_as<S>(at<S>(in, f, b)) - mean;
          var += d * d;
        }
        var /= C(n);
        C const inv_std = C(1) / d_sqrt(var + C(op.f0));
        for (int f = 0; f < n; f++) {
          C const xhat = (load_as<S>(at<S>(in, f, b)) - mean) * inv_std;
          store_as<S, C>(at<S>(out, f, b), params[op.woff + f] * xhat + params[op.boff + f]);
        }
        break;
      }
      case OP_SOFTMAX:
      case OP_LOG_SOFTMAX: {  // ponni_Softmax.h:45-56, ponni_LogSoftmax.h:45-57
        int const n = op.n_in;
        C mx = load_as<S>(at<S>(in, 0, b));
        for (int f = 1; f < n; f++) {
          C const v = load_as<S>(at<S>(in, f, b));
          mx = v > mx ? v : mx;
        }
        C sum = C(0);
        for (int f = 0; f < n; f++) sum += d_exp(load_as<S>(at<S>(in, f, b)) - mx);
        if (op.code == OP_SOFTMAX) {
          for (int f = 0; f < n; f++)
            store_as<S, C>(at<S>(out, f, b), d_exp(load_as<S>(at<S>(in, f, b)) - mx) / sum);
        } else {
          C const lse = d_log(sum) + mx;
          for (int f = 0; f < n; f++) store_as<S, C>(at<S>(out, f, b), load_as<S>(at<S>(in, f, b)) - lse);
        }
        break;
      }
      case OP_MIN_MAX: {  // ponni_MinMaxNorm.h:67-84
        int const n = op.n_in;
        C lo = load_as<S>(at<S>(in, 0, b));
        C hi = lo;
        for (int f = 1; f < n; f++) {
          C const v = load_as<S>(at<S>(in, f, b));
          if (v < lo) lo = v;
          if (v > hi) hi = v;
        }
        C const scale = (C(op.f1) - C(op.f0)) / ((hi - lo) + C(op.f2));
        for (int f = 0; f < n; f++)
          store_as<S, C>(at<S>(out, f, b), C(op.f0) + (load_as<S>(at<S>(in, f, b)) - lo) * scale);
        break;
      }
      case OP_SAVE: {  // ponni_Save_State.h:57-67; a leading save also fills tmp1
        for (int f = 0; f < op.n_out; f++) {
          S const v = *at<S>(in, f, b);
          *at<S>(out, f, b) = v;
          if (op.aux) *at<S>(buf.fixed[BUF_TMP1], f, b) = v;
        }
        break;
      }
      case OP_ADD: {  // ponni_Binop_Add.h:57-68
        View2 const sv = slot_view<S>(buf, op.slot);
        for (int f = 0; f < op.n_out; f++)
          store_as<S, C>(at<S>(out, f, b), load_as<S>(at<S>(in, f, b)) + load_as<S>(at<S>(sv, f, b)));
        break;
      }
      case OP_CONCAT: {  // ponni_Binop_Concatenate.h:63-86
        View2 const sv = slot_view<S>(buf, op.slot);
        int const n1 = op.n_in;
        int const n2 = op.n_out - op.n_in;
        if (op.aux) {
          // Rows below n1 keep the current state; an in-place write is safe.
          for (int f = n1; f < op.n_out; f++) *at<S>(out, f, b) = *at<S>(sv, f - n1, b);
          if (out.base != in.base)
            for (int f = 0; f < n1; f++) *at<S>(out, f, b) = *at<S>(in, f, b);
        } else {
          // [saved; current]: move the current rows up first (descending) so an
          // in-place write never reads an overwritten row.
          for (int f = op.n_out - 1; f >= n2; f--) *at<S>(out, f, b) = *at<S>(in, f - n2, b);
          for (int f = 0; f < n2; f++) *at<S>(out, f, b) = *at<S>(sv, f, b);
        }
        break;
      }
      case OP_PROJ_ADD: {  // ponni_Binop_Projection_Add.h:81-95
        View2 const sv = slot_view<S>(buf, op.slot);
        int const nsave = op.aux;
        int const n = op.n_out;
        C const* w = params + op.woff;
        for (int i = 0; i < n; i++) {
          C proj = params[op.boff + i];
          for (int k = 0; k < nsave; k++) proj += w[int64_t(k) * n + i] * load_as<S>(at<S>(sv, k, b));
          store_as<S, C>(at<S>(out, i, b), load_as<S>(at<S>(in, i, b)) + proj);
        }
        break;
      }
      case OP_EXTERNAL: {
        View2 const sv = slot_view<S>(buf, op.slot);
        ext(op.aux, op.boff, in, out, sv, op.n_in, op.n_out, b);
        if (op.boff & EXT_ALSO_TMP1) ext(op.aux, op.boff, in, buf.fixed[BUF_TMP1], sv, op.n_in, op.n_out, b);
        break;
      }
      case OP_LOAD: {  // the state becomes a saved one
        for (int f = 0; f < op.n_out; f++) *at<S>(out, f, b) = *at<S>(in, f, b);
        break;
      }
      case OP_BINARY: {  // emitter.py:735-741 with scalar-or-exact broadcasting
        View2 const sv = slot_view<S>(buf, op.slot);
        int const bop = op.aux & 0xff;
        bool const saved_left = op.aux & BIN_SAVED_LEFT;
        C const s0 = load_as<S>(at<S>(in, 0, b));
        C const v0 = load_as<S>(at<S>(sv, 0, b));
        for (int f = 0; f < op.n_out; f++) {
          C const a = (op.aux & BIN_STATE_SCALAR) ? s0 : load_as<S>(at<S>(in, f, b));
          C const c = (op.aux & BIN_SAVED_SCALAR) ? v0 : load_as<S>(at<S>(sv, f, b));
          store_as<S, C>(at<S>(out, f, b), saved_left ? apply_binary<C>(bop, c, a) : apply_binary<C>(bop, a, c));
        }
        break;
      }
      case OP_SELECT: {  // interpreter.py:178-183 Where / CompareSelect: cond != 0 ? a : b
        // Operand k comes from the state, a saved slot or a constant vector;
        // a one-feature operand is read once, before an in-place write.
        View2 const s1 = slot_view<S>(buf, op.slot);
        View2 const s2 = slot_view<S>(buf, op.f0 >= 0 ? static_cast<int>(op.f0) : op.slot);
        int const scalar_bits[3] = {SEL_COND_SCALAR, SEL_A_SCALAR, SEL_B_SCALAR};
        int coff = op.woff;
        C const* cvec[3] = {nullptr, nullptr, nullptr};
        View2 src[3];
        C first[3];
        for (int k = 0; k < 3; k++) {
          int const code = sel_src(op.aux, k);
          src[k] = code == 0 ? in : code == 1 ? s1 : s2;
          if (code == 3) {
            cvec[k] = params + coff;
            coff = op.boff;
          }
          first[k] = cvec[k] ? cvec[k][0] : load_as<S>(at<S>(src[k], 0, b));
        }
        for (int f = 0; f < op.n_out; f++) {
          C v[3];
          for (int k = 0; k < 3; k++)
            v[k] = (op.aux & scalar_bits[k]) ? first[k] : cvec[k] ? cvec[k][f] : load_as<S>(at<S>(src[k], f, b));
          store_as<S, C>(at<S>(out, f, b), apply_select<C>(v[0], v[1], v[2]));
        }
        break;
      }
      case OP_REDUCE: {  // emitter.py:475-547
        int const n = op.n_in;
        C r;
        if (op.aux == PONNI_REDUCE_MAX || op.aux == PONNI_REDUCE_MIN || op.aux == PONNI_REDUCE_LOG_SUM_EXP) {
          bool const mn = op.aux == PONNI_REDUCE_MIN;
          // 16-bit plans follow the generated half2 path, which keeps the
          // running value only if it compares past the next one
          // (TwoHalf::maximum(reduction, value), emitter.py:578-592): the
          // two orders differ only in where a NaN ends up.
          constexpr bool h2 = sizeof(S) == 2;
          r = load_as<S>(at<S>(in, 0, b));
          for (int f = 1; f < n; f++) {
            C const v = load_as<S>(at<S>(in, f, b));
            if (h2) r = mn ? (r < v ? r : v) : (r > v ? r : v);
            else r = mn ? (v < r ? v : r) : (v > r ? v : r);
          }
          if (op.aux == PONNI_REDUCE_LOG_SUM_EXP) {
            C sum = C(0);
            for (int f = 0; f < n; f++) sum += d_exp(load_as<S>(at<S>(in, f, b)) - r);
            r = __builtin_isinf(r) ? r : r + d_log(sum);
          }
        } else {
          r = op.aux == PONNI_REDUCE_PROD ? C(1) : C(0);
          for (int f = 0; f < n; f++) {
            C const v = load_as<S>(at<S>(in, f, b));
            switch (op.aux) {
              case PONNI_REDUCE_L1: r += d_abs(v); break;
              case PONNI_REDUCE_L2:
              case PONNI_REDUCE_SUM_SQUARE: r += v * v; break;
              case PONNI_REDUCE_PROD: r *= v; break;
              default: r += v; break;
            }
          }
          if (op.aux == PONNI_REDUCE_MEAN) r /= C(n);
          else if (op.aux == PONNI_REDUCE_L2) r = d_sqrt(r);
          else if (op.aux == PONNI_REDUCE_LOG_SUM) r = d_log(r);
        }
        store_as<S, C>(at<S>(out, 0, b), r);
        break;
      }
      default:
        break;
    }
  }
}

// The ops of a plan's program in order, for sample b.
template <class S, class Ext = NoExternal>
__host__ __device__ inline void run_ops(Op const* __restrict__ ops, int num_ops, Step const* __restrict__ steps,
                                        typename Compute<S>::type const* __restrict__ params,
                                        Bufs const& buf, int64_t b, Ext const& ext = Ext()) {
  for (int o = 0; o < num_ops; o++) run_op<S, Ext>(ops[o], steps, params, buf, b, ext);
}

// The same for a program known at compile time: Program::ops / ::steps are
// constexpr arrays (ponni_plan_program_source), each op expanded in place
// (the op is a constant expression, so its switch and sizes fold).
template <class S, class Program, int I, class Ext>
__host__ __device__ __attribute__((always_inline)) inline void run_program_op(
    typename Compute<S>::type const* __restrict__ params, Bufs const& buf, int64_t b,
    Ext const& ext) {
  constexpr Op op = Program::ops[I];
  run_op<S, Ext>(op, Program::steps, params, buf, b, ext);
}
template <class S, class Program, class Ext, int... I>
__host__ __device__ inline void run_program(typename Compute<S>::type const* __restrict__ params,
                                            Bufs const& buf, int64_t b, Ext const& ext,
                                            std::integer_sequence<int, I...>) {
  (run_program_op<S, Program, I, Ext>(params, buf, b, ext), ...);
}

}  // namespace ponni_hip
