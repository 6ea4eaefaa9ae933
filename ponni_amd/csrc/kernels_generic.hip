// GENERIC kernel family: one sample per lane, every intermediate state
// materialized in HBM scratch (tmp1 / tmp2 / saved slots) exactly where the
// reference's traverse_mixed_batch_parallel materializes it
// (src/ponni_Inference.h:453-555).  It runs any valid chain at any width and
// in F32, F64, F16 or BF16 storage; F16/BF16 compute in fp32.
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "generic_ops.h"
#include "plan.h"

namespace ponni_hip {

template <> __host__ __device__ inline float load_as<__half>(__half const* p) { return __half2float(*p); }
template <> __host__ __device__ inline float load_as<__hip_bfloat16>(__hip_bfloat16 const* p) { return __bfloat162float(*p); }
template <> __host__ __device__ inline void store_as<__half, float>(__half* p, float v) { *p = __float2half_rn(v); }
template <> __host__ __device__ inline void store_as<__hip_bfloat16, float>(__hip_bfloat16* p, float v) {
  *p = __float2bfloat16(v);
}

namespace {

template <class S>
__global__ __launch_bounds__(256) void generic_forward(LaunchArgs args) {
  using C = typename Compute<S>::type;
  int64_t const b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= args.batch) return;
  Bufs buf;
#pragma unroll
  for (int i = 0; i < BUF_SAVED; i++) buf.fixed[i] = View2{static_cast<char*>(args.buffers[i]), args.buffer_ld[i]};
  buf.saved = View2{static_cast<char*>(args.buffers[BUF_SAVED]), args.buffer_ld[BUF_SAVED]};
  buf.slot_row = args.slot_rows;
  run_ops<S>(args.ops, args.num_ops, args.steps, static_cast<C const*>(args.params), buf, b);
}

// ---- LAYERED: one dense block over the whole batch on the matrix cores ----
// out[f, b] = epilogue_f(sum_k W[k][f] in[k, b]) for a dense op of the GENERIC
// op list (W in the GENERIC packing, [n_in][n_out]; a generated Dense's bias
// seeds the sum), the other ops of the list running on generic_forward
// between such launches.  Tiles of 128 output features x 128 columns per
// 256-lane workgroup (each wave 64 x 64: 4 x 4 MFMA tiles), the contraction
// in steps of 16 features staged through LDS in the compute type (fp32 for
// fp32 / fp16 / bf16 storage, fp64 for fp64), the next step's global loads
// in flight while this step's MFMAs run.
template <class C> struct DenseMfma;
template <> struct DenseMfma<float> {
  typedef float V4 __attribute__((ext_vector_type(4)));
  __device__ static V4 op(float a, float b, V4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }
  // output row of element e in lane group g
  __device__ static int row(int g, int e) { return 4 * g + e; }
};
template <> struct DenseMfma<double> {
  typedef double V4 __attribute__((ext_vector_type(4)));
  __device__ static V4 op(double a, double b, V4 c) { return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0); }
  // (v_mfma_f64_16x16x4f64 returns the 4x4 row blocks transposed)
  __device__ static int row(int g, int e) { return 4 * e + g; }
};

constexpr int kLayeredOut = 128, kLayeredCols = 128, kLayeredK = 16, kLayeredPad = 16;

template <class S>
__global__ __launch_bounds__(256) void layered_dense(DenseArgs a) {
  using C = typename Compute<S>::type;
  using M = DenseMfma<C>;
  using V4 = typename M::V4;
  constexpr int BO = kLayeredOut, BB = kLayeredCols, KS = kLayeredK;
  __shared__ C As[2][KS][BO + kLayeredPad];
  __shared__ C Bs[2][KS][BB + kLayeredPad];
  int const tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15, wave = tid >> 6;
  int const wo = wave >> 1, wb = wave & 1;
  // Consecutive workgroups take the output blocks of one column block, so
  // its input tile is read from HBM once and then from L2.
  int const out_blocks = (a.n_out + BO - 1) / BO;
  int64_t const col0 = int64_t(blockIdx.x / out_blocks) * BB;
  int const out0 = int(blockIdx.x % out_blocks) * BO;
  C const* __restrict__ P = static_cast<C const*>(a.params);
  C const* __restrict__ W = P + a.woff;
  S const* __restrict__ X = static_cast<S const*>(a.x);
  V4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      int const f = out0 + 64 * wo + 16 * i + M::row(g, e);
      C const seed = a.bias_first && f < a.n_out ? P[a.steps[a.epi_begin].off + f] : C(0);
#pragma unroll
      for (int j = 0; j < 4; j++) acc[i][j][e] = seed;
    }
  // Staging: element idx = 256 i + tid of a step's 16 x 128 tiles is row
  // idx / 128, column idx % 128 (consecutive lanes, consecutive columns).
  C ra[8], rb[8];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      int const idx = 256 * i + tid, r = idx >> 7, cc = idx & 127, k = k0 + r;
      ra[i] = k < a.n_in && out0 + cc < a.n_out ? W[int64_t(k) * a.n_out + out0 + cc] : C(0);
      rb[i] = k < a.n_in && col0 + cc < a.batch ? load_as<S>(X + int64_t(k) * a.ldx + col0 + cc) : C(0);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      int const idx = 256 * i + tid, r = idx >> 7, cc = idx & 127;
      As[buf][r][cc] = ra[i];
      Bs[buf][r][cc] = rb[i];
    }
  };
  int const steps = (a.n_in + KS - 1) / KS;
  fetch(0);
  stash(0);
  __syncthreads();
  for (int s = 0; s < steps; s++) {
    int const buf = s & 1;
    if (s + 1 < steps) fetch((s + 1) * KS);
#pragma unroll
    for (int kk = 0; kk < KS / 4; kk++) {
      C av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) av[i] = As[buf][4 * kk + g][64 * wo + 16 * i + c];
#pragma unroll
      for (int j = 0; j < 4; j++) bv[j] = Bs[buf][4 * kk + g][64 * wb + 16 * j + c];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = M::op(av[i], bv[j], acc[i][j]);
    }
    // (buf ^ 1 was last read in step s - 1, which the barrier below ended)
    if (s + 1 < steps) stash(buf ^ 1);
    __syncthreads();
  }
  S* __restrict__ Y = static_cast<S*>(a.y);
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      int64_t const col = col0 + 64 * wb + 16 * j + c;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        int const f = out0 + 64 * wo + 16 * i + M::row(g, e);
        if (f >= a.n_out || col >= a.batch) continue;
        C v = acc[i][j][e];
        for (int k = a.bias_first; k < a.epi_count; k++) {  // ponni_Inference.h:431-444
          Step const st = a.steps[a.epi_begin + k];
          C const bias = act_has_param(st.act) ? P[st.off + f] : C(0);
          v = apply_step<C>(st.act, v, bias, C(st.a), C(st.b));
        }
        store_as<S, C>(Y + int64_t(f) * a.ldy + col, v);
      }
    }
}

}  // namespace

hipError_t launch_layered_dense(int dtype, DenseArgs const& a, hipStream_t stream) {
  if (a.batch <= 0) return hipSuccess;
  dim3 const block(256);
  int64_t const blocks = (a.batch + kLayeredCols - 1) / kLayeredCols * ((a.n_out + kLayeredOut - 1) / kLayeredOut);
  if (blocks > INT32_MAX) return hipErrorInvalidValue;
  dim3 const grid(static_cast<unsigned>(blocks));
  switch (dtype) {
    case PONNI_F64: hipLaunchKernelGGL(layered_dense<double>, grid, block, 0, stream, a); break;
    case PONNI_F16: hipLaunchKernelGGL(layered_dense<__half>, grid, block, 0, stream, a); break;
    case PONNI_BF16: hipLaunchKernelGGL(layered_dense<__hip_bfloat16>, grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL(layered_dense<float>, grid, block, 0, stream, a); break;
  }
  return hipGetLastError();
}

hipError_t launch_generic(int dtype, LaunchArgs const& args, hipStream_t stream) {
  dim3 const block(256);
  dim3 const grid(static_cast<unsigned>((args.batch + 255) / 256));
  switch (dtype) {
    case PONNI_F64: launch_kernel(generic_forward<double>, grid, block, 0, stream, args, args); break;
    case PONNI_F16: launch_kernel(generic_forward<__half>, grid, block, 0, stream, args, args); break;
    case PONNI_BF16: launch_kernel(generic_forward<__hip_bfloat16>, grid, block, 0, stream, args, args); break;
    default: launch_kernel(generic_forward<float>, grid, block, 0, stream, args, args); break;
  }
  return hipGetLastError();
}

}  // namespace ponni_hip
