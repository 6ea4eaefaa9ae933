// NARROW kernel family: one sample per lane with the whole state vector in
// registers.  For chains no wider than 16 features (e.g. the reference's
// README 2->3->1 network) every layer -- dense, pointwise, barrier and saved
// states -- runs on registers, so HBM sees only the input read and the output
// write.  Weights are zero-padded to W x W and read with uniform (scalar)
// loads; the op loop is uniform control flow.
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "plan.h"
#include "pointwise.h"

namespace ponni_hip {
namespace {

template <class S> __device__ inline float to_f(S v) { return static_cast<float>(v); }
template <> __device__ inline float to_f<__half>(__half v) { return __half2float(v); }
template <> __device__ inline float to_f<__hip_bfloat16>(__hip_bfloat16 v) { return __bfloat162float(v); }
template <class S> __device__ inline S from_f(float v) { return static_cast<S>(v); }
template <> __device__ inline __half from_f<__half>(float v) { return __float2half_rn(v); }
template <> __device__ inline __hip_bfloat16 from_f<__hip_bfloat16>(float v) { return __float2bfloat16(v); }
// Rounding of a materialized state to the storage precision.
template <class S> __device__ inline float round_state(float v) { return to_f<S>(from_f<S>(v)); }
template <> __device__ inline float round_state<float>(float v) { return v; }

constexpr int kWaves = 4;

// One pointwise step over all W x P register values (bias per feature row).
template <int W, int P>
__device__ inline void apply_step_rows(Step const& sp, float const* __restrict__ prm, float (&v)[W][P]) {
  if (sp.act == ACT_BIAS) {
#pragma unroll
    for (int j = 0; j < W; j++) {
      float const bias = prm[sp.off + j];
#pragma unroll
      for (int p = 0; p < P; p++) v[j][p] += bias;
    }
    return;
  }
  map_activation<float>(sp.act, float(sp.a), float(sp.b), [&](auto&& f) {
#pragma unroll
    for (int j = 0; j < W; j++)
#pragma unroll
      for (int p = 0; p < P; p++) f(v[j][p]);
  });
}

// W: padded width; P: samples per lane (strided by 64 inside the wave tile);
// NS: saved-state slots held in registers.
template <class S, int W, int P, int NS>
__global__ __launch_bounds__(256) void narrow_forward(LaunchArgs a) {
  int const lane = threadIdx.x & 63;
  int const wave = threadIdx.x >> 6;
  int64_t const base = (int64_t(blockIdx.x) * kWaves + wave) * (64 * P) + lane;
  float const* __restrict__ prm = static_cast<float const*>(a.params);
  S const* __restrict__ x = static_cast<S const*>(a.x);
  S* __restrict__ y = static_cast<S*>(a.y);

  float st[W][P];
  float sv[NS > 0 ? NS : 1][W][P];
#pragma unroll
  for (int f = 0; f < W; f++) {
#pragma unroll
    for (int p = 0; p < P; p++) {
      int64_t const b = base + 64 * p;
      st[f][p] = (f < a.num_inputs && b < a.batch) ? to_f<S>(x[int64_t(f) * a.ld_x + b]) : 0.0f;
    }
  }
#pragma unroll
  for (int s = 0; s < (NS > 0 ? NS : 1); s++)
#pragma unroll
    for (int f = 0; f < W; f++)
#pragma unroll
      for (int p = 0; p < P; p++) sv[s][f][p] = 0.0f;

  for (int o = 0; o < a.num_ops; o++) {
    Op const op = a.ops[o];
    switch (op.code) {
      case OP_DENSE: {
        float acc[W][P];
        float const* w = prm + op.woff;
#pragma unroll
        for (int j = 0; j < W; j++) {
#pragma unroll
          for (int p = 0; p < P; p++) acc[j][p] = 0.0f;
#pragma unroll
          for (int k = 0; k < W; k++) {
            float const wk = w[k * W + j];
#pragma unroll
            for (int p = 0; p < P; p++) acc[j][p] += wk * st[k][p];
          }
        }
        for (int s = 0; s < op.epi_count; s++) apply_step_rows<W, P>(a.steps[op.epi_begin + s], prm, acc);
#pragma unroll
        for (int j = 0; j < W; j++)
#pragma unroll
          for (int p = 0; p < P; p++) st[j][p] = acc[j][p];
        break;
      }
      case OP_POINTWISE: {
        apply_step_rows<W, P>(a.steps[op.epi_begin], prm, st);
        break;
      }
      case OP_LAYER_NORM: {  // two-pass statistics, ponni_LayerNorm.h:82-98
        int const n = op.n_in;
#pragma unroll
        for (int p = 0; p < P; p++) {
          float mean = 0.0f;
#pragma unroll
          for (int f = 0; f < W; f++)
            if (f < n) mean += st[f][p];
          mean /= float(n);
          float var = 0.0f;
#pragma unroll
          for (int f = 0; f < W; f++)
            if (f < n) {
              float const d = st[f][p] - mean;
              var += d * d;
            }
          var /= float(n);
          float const inv_std = 1.0f / sqrtf(var + float(op.f0));
#pragma unroll
          for (int f = 0; f < W; f++) st[f][p] = prm[op.woff + f] * ((st[f][p] - mean) * inv_std) + prm[op.boff + f];
        }
        break;
      }
      case OP_SOFTMAX:
      case OP_LOG_SOFTMAX: {
        int const n = op.n_in;
#pragma unroll
        for (int p = 0; p < P; p++) {
          float mx = st[0][p];
#pragma unroll
          for (int f = 1; f < W; f++)
            if (f < n) mx = st[f][p] > mx ? st[f][p] : mx;
          float sum = 0.0f;
#pragma unroll
          for (int f = 0; f < W; f++)
            if (f < n) sum += expf(st[f][p] - mx);
          if (op.code == OP_SOFTMAX) {
#pragma unroll
            for (int f = 0; f < W; f++) st[f][p] = expf(st[f][p] - mx) / sum;
          } else {
            float const lse = logf(sum) + mx;
#pragma unroll
            for (int f = 0; f < W; f++) st[f][p] = st[f][p] - lse;
          }
        }
        break;
      }
      case OP_MIN_MAX: {
        int const n = op.n_in;
#pragma unroll
        for (int p = 0; p < P; p++) {
          float lo = st[0][p], hi = st[0][p];
#pragma unroll
          for (int f = 1; f < W; f++)
            if (f < n) {
              if (st[f][p] < lo) lo = st[f][p];
              if (st[f][p] > hi) hi = st[f][p];
            }
          float const scale = (float(op.f1) - float(op.f0)) / ((hi - lo) + float(op.f2));
#pragma unroll
          for (int f = 0; f < W; f++) st[f][p] = float(op.f0) + (st[f][p] - lo) * scale;
        }
        break;
      }
      case OP_SAVE: {
#pragma unroll
        for (int s = 0; s < NS; s++)
          if (s == op.slot)
#pragma unroll
            for (int f = 0; f < W; f++)
#pragma unroll
              for (int p = 0; p < P; p++) sv[s][f][p] = st[f][p];
        break;
      }
      case OP_ADD: {
#pragma unroll
        for (int s = 0; s < NS; s++)
          if (s == op.slot)
#pragma unroll
            for (int f = 0; f < W; f++)
#pragma unroll
              for (int p = 0; p < P; p++) st[f][p] += sv[s][f][p];
        break;
      }
      case OP_CONCAT: {
        // after: [state(n1); saved] ; otherwise [saved(n2); state]
        int const n1 = op.n_in;
        int const first = op.aux ? n1 : op.n_out - n1;  // rows taken from the leading operand
#pragma unroll
        for (int s = 0; s < NS; s++)
          if (s == op.slot) {
            float out[W][P];
#pragma unroll
            for (int f = 0; f < W; f++) {
#pragma unroll
              for (int p = 0; p < P; p++) out[f][p] = 0.0f;
#pragma unroll
              for (int q = 0; q < W; q++) {
                // Leading operand rows keep their index; trailing rows shift by `first`.
                if (q == f && f < first) {
#pragma unroll
                  for (int p = 0; p < P; p++) out[f][p] = op.aux ? st[q][p] : sv[s][q][p];
                }
                if (q + first == f) {
#pragma unroll
                  for (int p = 0; p < P; p++) out[f][p] = op.aux ? sv[s][q][p] : st[q][p];
                }
              }
            }
#pragma unroll
            for (int f = 0; f < W; f++)
#pragma unroll
              for (int p = 0; p < P; p++) st[f][p] = out[f][p];
          }
        break;
      }
      case OP_PROJ_ADD: {
#pragma unroll
        for (int s = 0; s < NS; s++)
          if (s == op.slot) {
            float const* w = prm + op.woff;
#pragma unroll
            for (int i = 0; i < W; i++) {
              float proj[P];
#pragma unroll
              for (int p = 0; p < P; p++) proj[p] = prm[op.boff + i];
#pragma unroll
              for (int k = 0; k < W; k++) {
                float const wk = w[k * W + i];
#pragma unroll
                for (int p = 0; p < P; p++) proj[p] += wk * sv[s][k][p];
              }
#pragma unroll
              for (int p = 0; p < P; p++) st[i][p] = st[i][p] + proj[p];
            }
          }
        break;
      }
      default:
        break;
    }
    // Keep padding rows at exactly zero and round the state to the storage
    // precision, as every materialization of the reference executor does.
#pragma unroll
    for (int f = 0; f < W; f++)
#pragma unroll
      for (int p = 0; p < P; p++) st[f][p] = f < op.n_out ? round_state<S>(st[f][p]) : 0.0f;
  }

#pragma unroll
  for (int f = 0; f < W; f++) {
    if (f < a.num_outputs) {
#pragma unroll
      for (int p = 0; p < P; p++) {
        int64_t const b = base + 64 * p;
        if (b < a.batch) y[int64_t(f) * a.ld_y + b] = from_f<S>(st[f][p]);
      }
    }
  }
}

template <class S, int W, int P>
hipError_t launch_w(int num_slots, LaunchArgs const& a, hipStream_t stream) {
  int64_t const per_block = int64_t(kWaves) * 64 * P;
  dim3 const grid(static_cast<unsigned>((a.batch + per_block - 1) / per_block));
  dim3 const block(kWaves * 64);
  if (num_slots == 0) launch_kernel(narrow_forward<S, W, P, 0>, grid, block, 0, stream, a, a);
  else if (num_slots == 1) launch_kernel(narrow_forward<S, W, P, 1>, grid, block, 0, stream, a, a);
  else launch_kernel(narrow_forward<S, W, P, 2>, grid, block, 0, stream, a, a);
  return hipGetLastError();
}

template <class S>
hipError_t launch_s(int width_class, int num_slots, LaunchArgs const& a, hipStream_t stream) {
  switch (width_class) {
    case 4: return launch_w<S, 4, 4>(num_slots, a, stream);
    case 8: return launch_w<S, 8, 2>(num_slots, a, stream);
    default: return launch_w<S, 16, 1>(num_slots, a, stream);
  }
}

}  // namespace

int narrow_width_class(int max_width) {
  if (max_width <= 4) return 4;
  if (max_width <= 8) return 8;
  if (max_width <= 16) return 16;
  return 0;
}

hipError_t launch_narrow(int dtype, int width_class, int num_slots, LaunchArgs const& a, hipStream_t stream) {
  switch (dtype) {
    case PONNI_F16: return launch_s<__half>(width_class, num_slots, a, stream);
    case PONNI_BF16: return launch_s<__hip_bfloat16>(width_class, num_slots, a, stream);
    default: return launch_s<float>(width_class, num_slots, a, stream);
  }
}

}  // namespace ponni_hip
