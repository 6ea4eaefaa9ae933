// MFMA kernel family (fp32), included once per width class by
// kernels_mfma_f32_mt*.hip.  A wave owns a tile of 32 batch columns and keeps
// the whole feature state of those columns in registers, laid out exactly as
// the D operand of v_mfma_f32_16x16x4f32:
//
//   st[m][n][v] (lane l, g = l/16, c = l%16)  <->  feature 16m + 4g + v,
//                                                 column  16n + c.
//
// A Matvec layer is the contraction Y[o, b] = sum_k W[k, o] X[k, b].  Feeding
// st[m][n][v] straight back as the B operand (B[k][j] lives in lane j + 16k)
// contracts features {16m + 4k + v : k = 0..3}; the host packs W into the
// matching A-fragment order (lane l, element v = W[16m + 4(l/16) + v][16mo +
// l%16]), so consecutive layers chain through registers with no LDS or HBM
// round trip.  Bias, activations, LayerNorm, softmax, residual saves/adds and
// projection skips all operate on the register tile; HBM sees the input read
// and the output write only.
#pragma once

#include <hip/hip_runtime.h>

#include "plan.h"
#include "pointwise.h"

namespace ponni_hip {
namespace mfma_f32 {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;   // waves per workgroup
constexpr int kNT = 2;      // 16-column tiles per wave

__device__ inline float xor_sum(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}
__device__ inline float xor_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}
__device__ inline float xor_min(float v) {
  v = fminf(v, __shfl_xor(v, 16));
  v = fminf(v, __shfl_xor(v, 32));
  return v;
}

// acc[mo][n] += sum over input tiles of W^T * src, for output tiles mo < mto.
// All A fragments of one output tile are fetched before its MFMAs, so the
// load latency is paid once per output tile rather than once per fragment.
template <int MT>
__device__ inline void dense_tiles(floatx4 (&acc)[MT][kNT], floatx4 const (&src)[MT][kNT],
                                   float const* __restrict__ wp, int mti, int mto, int lane) {
#pragma unroll
  for (int mo = 0; mo < MT; mo++) {
    if (mo < mto) {
      floatx4 w[MT];
#pragma unroll
      for (int m = 0; m < MT; m++)
        if (m < mti) w[m] = *reinterpret_cast<floatx4 const*>(wp + ((mo * mti + m) * 64 + lane) * 4);
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if (m < mti) {
#pragma unroll
          for (int v = 0; v < 4; v++)
#pragma unroll
            for (int n = 0; n < kNT; n++)
              acc[mo][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[m][v], src[m][n][v], acc[mo][n], 0, 0, 0);
        }
      }
    }
  }
}

// One pointwise step over the output tiles mo < mt (bias per feature row).
template <int MT>
__device__ inline void apply_step_tiles(Step const& sp, float const* __restrict__ prm, floatx4 (&t)[MT][kNT], int mt,
                                        int g) {
  if (sp.act == ACT_BIAS) {
#pragma unroll
    for (int mo = 0; mo < MT; mo++)
      if (mo < mt) {
        floatx4 const bias = *reinterpret_cast<floatx4 const*>(prm + sp.off + 16 * mo + 4 * g);
#pragma unroll
        for (int n = 0; n < kNT; n++) t[mo][n] += bias;
      }
    return;
  }
  map_activation<float>(sp.act, float(sp.a), float(sp.b), [&](auto&& f) {
#pragma unroll
    for (int mo = 0; mo < MT; mo++)
      if (mo < mt) {
#pragma unroll
        for (int n = 0; n < kNT; n++)
#pragma unroll
          for (int v = 0; v < 4; v++) {
            float e = t[mo][n][v];
            f(e);
            t[mo][n][v] = e;
          }
      }
  });
}

// LDS: when the packed parameters fit, each workgroup stages them in LDS once
// and then loops over column tiles (persistent), so every A fragment, bias and
// gamma is an LDS read; otherwise they stream from L2.
template <int MT, int NS, bool LDS>
__global__ __launch_bounds__(256) void mfma_forward_f32(LaunchArgs a) {
  extern __shared__ floatx4 lds_params[];
  int const lane = threadIdx.x & 63;
  int const wave = threadIdx.x >> 6;
  int const g = lane >> 4;
  int const c = lane & 15;
  float const* __restrict__ prm;
  if constexpr (LDS) {
    floatx4 const* src = static_cast<floatx4 const*>(a.params);
    int const n4 = static_cast<int>((a.param_count + 3) >> 2);
    for (int i = threadIdx.x; i < n4; i += blockDim.x) lds_params[i] = src[i];
    __syncthreads();
    prm = reinterpret_cast<float const*>(lds_params);
  } else {
    prm = static_cast<float const*>(a.params);
  }
  float const* __restrict__ x = static_cast<float const*>(a.x);
  float* __restrict__ y = static_cast<float*>(a.y);
  int64_t const tiles = (a.batch + kWaves * 16 * kNT - 1) / (kWaves * 16 * kNT);
  for (int64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
  int64_t const col0 = (tile * kWaves + wave) * (16 * kNT);

  floatx4 st[MT][kNT];
  floatx4 sv[NS > 0 ? NS : 1][MT][kNT];

  int const mt_in = (a.num_inputs + 15) >> 4;
#pragma unroll
  for (int m = 0; m < MT; m++)
#pragma unroll
    for (int n = 0; n < kNT; n++) {
      int64_t const b = col0 + 16 * n + c;
#pragma unroll
      for (int v = 0; v < 4; v++) {
        int const f = 16 * m + 4 * g + v;
        st[m][n][v] = (m < mt_in && f < a.num_inputs && b < a.batch) ? x[int64_t(f) * a.ld_x + b] : 0.0f;
      }
    }
#pragma unroll
  for (int s = 0; s < (NS > 0 ? NS : 1); s++)
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
      for (int n = 0; n < kNT; n++) sv[s][m][n] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int o = 0; o < a.num_ops; o++) {
    Op const op = a.ops[o];
    int const mt_out = (op.n_out + 15) >> 4;
    switch (op.code) {
      case OP_DENSE: {
        floatx4 acc[MT][kNT];
#pragma unroll
        for (int mo = 0; mo < MT; mo++)
#pragma unroll
          for (int n = 0; n < kNT; n++) acc[mo][n] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        dense_tiles<MT>(acc, st, prm + op.woff, (op.n_in + 15) >> 4, mt_out, lane);
        for (int s = 0; s < op.epi_count; s++) apply_step_tiles<MT>(a.steps[op.epi_begin + s], prm, acc, mt_out, g);
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
          for (int n = 0; n < kNT; n++) st[m][n] = acc[m][n];
        break;
      }
      case OP_POINTWISE: {
        apply_step_tiles<MT>(a.steps[op.epi_begin], prm, st, mt_out, g);
        break;
      }
      case OP_LAYER_NORM: {  // two-pass mean / biased variance, ponni_LayerNorm.h:82-98
        int const nf = op.n_in;
#pragma unroll
        for (int n = 0; n < kNT; n++) {
          float s = 0.0f;
#pragma unroll
          for (int m = 0; m < MT; m++)
#pragma unroll
            for (int v = 0; v < 4; v++)
              if (16 * m + 4 * g + v < nf) s += st[m][n][v];
          float const mean = xor_sum(s) / float(nf);
          float q = 0.0f;
#pragma unroll
          for (int m = 0; m < MT; m++)
#pragma unroll
            for (int v = 0; v < 4; v++)
              if (16 * m + 4 * g + v < nf) {
                float const d = st[m][n][v] - mean;
                q += d * d;
              }
          float const var = xor_sum(q) / float(nf);
          float const inv_std = 1.0f / sqrtf(var + float(op.f0));
#pragma unroll
          for (int m = 0; m < MT; m++) {
            if (m < mt_out) {
              floatx4 const gm = *reinterpret_cast<floatx4 const*>(prm + op.woff + 16 * m + 4 * g);
              floatx4 const bt = *reinterpret_cast<floatx4 const*>(prm + op.boff + 16 * m + 4 * g);
#pragma unroll
              for (int v = 0; v < 4; v++) st[m][n][v] = gm[v] * ((st[m][n][v] - mean) * inv_std) + bt[v];
            }
          }
        }
        break;
      }
      case OP_SOFTMAX:
      case OP_LOG_SOFTMAX: {
        int const nf = op.n_in;
#pragma unroll
        for (int n = 0; n < kNT; n++) {
          float mx = -INFINITY;
#pragma unroll
          for (int m = 0; m < MT; m++)
#pragma unroll
            for (int v = 0; v < 4; v++)
              if (16 * m + 4 * g + v < nf) mx = fmaxf(mx, st[m][n][v]);
          mx = xor_max(mx);
          float s = 0.0f;
#pragma unroll
          for (int m = 0; m < MT; m++)
#pragma unroll
            for (int v = 0; v < 4; v++)
              if (16 * m + 4 * g + v < nf) s += expf(st[m][n][v] - mx);
          s = xor_sum(s);
          if (op.code == OP_SOFTMAX) {
#pragma unroll
            for (int m = 0; m < MT; m++)
#pragma unroll
              for (int v = 0; v < 4; v++) st[m][n][v] = expf(st[m][n][v] - mx) / s;
          } else {
            float const lse = logf(s) + mx;
#pragma unroll
            for (int m = 0; m < MT; m++)
#pragma unroll
              for (int v = 0; v < 4; v++) st[m][n][v] = st[m][n][v] - lse;
          }
        }
        break;
      }
      case OP_MIN_MAX: {
        int const nf = op.n_in;
#pragma unroll
        for (int n = 0; n < kNT; n++) {
          float lo = INFINITY, hi = -INFINITY;
#pragma unroll
          for (int m = 0; m < MT; m++)
#pragma unroll
            for (int v = 0; v < 4; v++)
              if (16 * m + 4 * g + v < nf) {
                lo = fminf(lo, st[m][n][v]);
                hi = fmaxf(hi, st[m][n][v]);
              }
          lo = xor_min(lo);
          hi = xor_max(hi);
          // The reference's running minimum / maximum starts from feature 0
          // and replaces it only on a strict comparison: a NaN there makes
          // both NaN, a NaN elsewhere is passed over (as fminf / fmaxf do).
          float const x0 = st[0][n][0];  // feature 0: lane group 0, element 0
          if (xor_max(g == 0 && x0 != x0 ? 1.0f : 0.0f) != 0.0f) lo = hi = __builtin_nanf("");
          float const scale = (float(op.f1) - float(op.f0)) / ((hi - lo) + float(op.f2));
#pragma unroll
          for (int m = 0; m < MT; m++)
#pragma unroll
            for (int v = 0; v < 4; v++) st[m][n][v] = float(op.f0) + (st[m][n][v] - lo) * scale;
        }
        break;
      }
      case OP_SAVE: {
#pragma unroll
        for (int s = 0; s < NS; s++)
          if (s == op.slot)
#pragma unroll
            for (int m = 0; m < MT; m++)
#pragma unroll
              for (int n = 0; n < kNT; n++) sv[s][m][n] = st[m][n];
        break;
      }
      case OP_ADD: {
#pragma unroll
        for (int s = 0; s < NS; s++)
          if (s == op.slot)
#pragma unroll
            for (int m = 0; m < MT; m++)
#pragma unroll
              for (int n = 0; n < kNT; n++) st[m][n] += sv[s][m][n];
        break;
      }
      case OP_CONCAT: {
        // Tile-granular: the leading operand keeps tiles [0, t), the trailing
        // operand moves up by t tiles (the planner requires 16 | leading rows).
        int const lead = op.aux ? op.n_in : op.n_out - op.n_in;
        int const t = lead >> 4;
#pragma unroll
        for (int s = 0; s < NS; s++)
          if (s == op.slot) {
            floatx4 out[MT][kNT];
#pragma unroll
            for (int m = 0; m < MT; m++) {
#pragma unroll
              for (int n = 0; n < kNT; n++) out[m][n] = op.aux ? st[m][n] : sv[s][m][n];
#pragma unroll
              for (int q = 0; q < MT; q++)
                if (q + t == m)
#pragma unroll
                  for (int n = 0; n < kNT; n++) out[m][n] = op.aux ? sv[s][q][n] : st[q][n];
            }
#pragma unroll
            for (int m = 0; m < MT; m++)
#pragma unroll
              for (int n = 0; n < kNT; n++) st[m][n] = out[m][n];
          }
        break;
      }
      case OP_PROJ_ADD: {  // out = in + (b + W^T saved), ponni_Binop_Projection_Add.h:90-94
#pragma unroll
        for (int s = 0; s < NS; s++)
          if (s == op.slot) {
            floatx4 acc[MT][kNT];
#pragma unroll
            for (int mo = 0; mo < MT; mo++) {
              floatx4 bias = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
              if (mo < mt_out) bias = *reinterpret_cast<floatx4 const*>(prm + op.boff + 16 * mo + 4 * g);
#pragma unroll
              for (int n = 0; n < kNT; n++) acc[mo][n] = bias;
            }
            dense_tiles<MT>(acc, sv[s], prm + op.woff, (op.aux + 15) >> 4, mt_out, lane);
#pragma unroll
            for (int m = 0; m < MT; m++)
#pragma unroll
              for (int n = 0; n < kNT; n++) st[m][n] = st[m][n] + acc[m][n];
          }
        break;
      }
      default:
        break;
    }
    // Rows past the state width stay exactly zero (padding of the K dimension).
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
      for (int n = 0; n < kNT; n++)
#pragma unroll
        for (int v = 0; v < 4; v++)
          if (16 * m + 4 * g + v >= op.n_out) st[m][n][v] = 0.0f;
  }

  int const mt_y = (a.num_outputs + 15) >> 4;
#pragma unroll
  for (int m = 0; m < MT; m++) {
    if (m < mt_y) {
#pragma unroll
      for (int n = 0; n < kNT; n++) {
        int64_t const b = col0 + 16 * n + c;
#pragma unroll
        for (int v = 0; v < 4; v++) {
          int const f = 16 * m + 4 * g + v;
          if (f < a.num_outputs && b < a.batch) y[int64_t(f) * a.ld_y + b] = st[m][n][v];
        }
      }
    }
  }
  }  // column tiles
}

// Largest packed parameter block staged in LDS (two workgroups per CU fit).
constexpr int64_t kLdsParamBytes = 64 * 1024;

template <int MT, int NS>
hipError_t launch_ns(LaunchArgs const& a, hipStream_t stream) {
  int64_t const per_block = int64_t(kWaves) * 16 * kNT;
  int64_t const tiles = (a.batch + per_block - 1) / per_block;
  dim3 const block(kWaves * 64);
  size_t const bytes = static_cast<size_t>((a.param_count + 3) / 4 * 16);
  if (int64_t(bytes) <= kLdsParamBytes) {
    int dev = 0, cus = 0, per_cu = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess)
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, mfma_forward_f32<MT, NS, true>, kWaves * 64, bytes);
    if (e != hipSuccess) return e;
    int64_t const resident = int64_t(cus) * (per_cu > 0 ? per_cu : 1);
    dim3 const grid(static_cast<unsigned>(tiles < resident ? tiles : resident));
    launch_kernel(mfma_forward_f32<MT, NS, true>, grid, block, uint32_t(bytes), stream, a, a);
  } else {
    dim3 const grid(static_cast<unsigned>(tiles));
    launch_kernel(mfma_forward_f32<MT, NS, false>, grid, block, 0, stream, a, a);
  }
  return hipGetLastError();
}

template <int MT>
hipError_t launch(int num_slots, LaunchArgs const& a, hipStream_t stream) {
  if (num_slots == 0) return launch_ns<MT, 0>(a, stream);
  if (num_slots == 1) return launch_ns<MT, 1>(a, stream);
  return launch_ns<MT, 2>(a, stream);
}

}  // namespace mfma_f32
}  // namespace ponni_hip
