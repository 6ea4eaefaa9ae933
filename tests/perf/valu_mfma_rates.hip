// Instruction-rate probe for the 16-bit FUSED kernels on gfx950 (not a test:
// built and run by hand, its output summarized with the command that made
// it).  It answers two questions the c4 kernel's design rests on:
//
//  1. What a Tanh costs: throughput of v_fma_f32, v_exp_f32, v_rcp_f32, the
//     Tanh chain (2^x, 1 + e, 1 / d, scale), v_pk_fma_f16, and the fp16
//     transcendentals v_rcp_f16 / v_exp_f16 on both halves of a pair.
//  2. Whether VALU work runs in the shadow of v_mfma_f32_16x16x32_f16: each
//     thread issues 4 independent MFMAs per iteration with 0, 16 FMAs or 4 / 8
//     Tanh chains between them, at 1, 2 and 4 waves per SIMD.
//
// Every kernel writes one float per thread into a buffer sized for the
// largest launch; the values are discarded.
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       tests/perf/valu_mfma_rates.hip -o /tmp/valu_mfma_rates && /tmp/valu_mfma_rates
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdio>

namespace {

constexpr int kIter = 2048;
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

__device__ inline float tanh_chain(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x)) * -0.5f;
}

// Part 1: 8 independent chains of one operation per thread.
template <int OP>
__global__ __launch_bounds__(256) void rate(float* out, float seed) {
  float a[8];
  for (int j = 0; j < 8; j++) a[j] = seed + 0.001f * (threadIdx.x + j);
  if constexpr (OP <= 3) {
    for (int i = 0; i < kIter; i++) {
#pragma unroll
      for (int j = 0; j < 8; j++) {
        if constexpr (OP == 0) a[j] = __builtin_fmaf(a[j], 0.999f, 0.0001f);
        if constexpr (OP == 1) a[j] = __builtin_amdgcn_exp2f(a[j]) * -0.25f;
        if constexpr (OP == 2) a[j] = __builtin_amdgcn_rcpf(a[j]) + 0.5f;
        if constexpr (OP == 3) a[j] = tanh_chain(a[j]);
      }
    }
    float s = 0;
    for (int j = 0; j < 8; j++) s += a[j];
    out[blockIdx.x * 256 + threadIdx.x] = s;
  } else {
    __half2 h[8];
    for (int j = 0; j < 8; j++) h[j] = __floats2half2_rn(a[j], a[j] + 0.5f);
    __half2 const c1 = __floats2half2_rn(0.999f, 0.999f), c2 = __floats2half2_rn(0.0001f, 0.0001f);
    for (int i = 0; i < kIter; i++) {
#pragma unroll
      for (int j = 0; j < 8; j++) {
        if constexpr (OP == 4) h[j] = __hfma2(h[j], c1, c2);
        if constexpr (OP == 5) h[j] = __halves2half2(hrcp(__low2half(h[j])), hrcp(__high2half(h[j])));
        if constexpr (OP == 6) h[j] = __halves2half2(hexp2(__low2half(h[j])), hexp2(__high2half(h[j])));
      }
    }
    float s = 0;
    for (int j = 0; j < 8; j++) s += __low2float(h[j]) + __high2float(h[j]);
    out[blockIdx.x * 256 + threadIdx.x] = s;
  }
}

// Part 2: NM MFMAs per iteration, NV operations of kind K (0 FMA, 1 Tanh
// chain) after each; NM == 0 runs 4 NV operations per iteration alone.
template <int NM, int NV, int K>
__global__ __launch_bounds__(256) void overlap(float* out, float seed) {
  f4 acc[4];
  for (int j = 0; j < 4; j++) acc[j] = f4{seed, 0, 0, 0};
  h8 a, b;
  for (int j = 0; j < 8; j++) {
    a[j] = static_cast<_Float16>(0.01f * (threadIdx.x + j));
    b[j] = static_cast<_Float16>(0.02f * j);
  }
  float v[8];
  for (int j = 0; j < 8; j++) v[j] = seed + 0.001f * (threadIdx.x + j);
  for (int i = 0; i < kIter; i++) {
#pragma unroll
    for (int m = 0; m < NM; m++) {
      acc[m % 4] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[m % 4], 0, 0, 0);
#pragma unroll
      for (int q = 0; q < NV; q++) {
        float& x = v[(m * NV + q) % 8];
        x = K == 0 ? __builtin_fmaf(x, 0.999f, 0.0001f) : tanh_chain(x);
      }
    }
    if constexpr (NM == 0) {
#pragma unroll
      for (int q = 0; q < NV * 4; q++) {
        float& x = v[q % 8];
        x = K == 0 ? __builtin_fmaf(x, 0.999f, 0.0001f) : tanh_chain(x);
      }
    }
  }
  float s = 0;
  for (int j = 0; j < 4; j++) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  for (int j = 0; j < 8; j++) s += v[j];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

template <class Launch>
float time_ms(Launch launch) {
  hipEvent_t a, b;
  (void)hipEventCreate(&a);
  (void)hipEventCreate(&b);
  launch();  // warm-up
  (void)hipEventRecord(a);
  launch();
  (void)hipEventRecord(b);
  (void)hipEventSynchronize(b);
  float ms = 0;
  (void)hipEventElapsedTime(&ms, a, b);
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  return ms;
}

}  // namespace

int main() {
  int device_cus = 0;
  (void)hipDeviceGetAttribute(&device_cus, hipDeviceAttributeMultiprocessorCount, 0);
  int const simds = 4 * device_cus;
  int const max_blocks = device_cus * 8;
  float* d = nullptr;
  if (hipMalloc(&d, sizeof(float) * max_blocks * 256) != hipSuccess) return 1;

  // Part 1: 8 waves per SIMD (8 blocks of 4 waves per CU).
  int const blocks = device_cus * 8;
  double const per_simd = double(blocks) * 4 * kIter * 8 / simds;  // wave-instructions of the op per SIMD
  char const* names[] = {"v_fma_f32", "v_exp_f32 + mul", "v_rcp_f32 + add", "tanh chain (exp, add, rcp, mul)",
                         "v_pk_fma_f16 (2 elements)", "2 v_rcp_f16 (a pair)", "2 v_exp_f16 (a pair)"};
  float ms[7];
  ms[0] = time_ms([&] { rate<0><<<blocks, 256>>>(d, 0.5f); });
  ms[1] = time_ms([&] { rate<1><<<blocks, 256>>>(d, 0.5f); });
  ms[2] = time_ms([&] { rate<2><<<blocks, 256>>>(d, 0.5f); });
  ms[3] = time_ms([&] { rate<3><<<blocks, 256>>>(d, 0.5f); });
  ms[4] = time_ms([&] { rate<4><<<blocks, 256>>>(d, 0.5f); });
  ms[5] = time_ms([&] { rate<5><<<blocks, 256>>>(d, 0.5f); });
  ms[6] = time_ms([&] { rate<6><<<blocks, 256>>>(d, 0.5f); });
  printf("part 1: throughput, 8 waves per SIMD (%d SIMDs)\n", simds);
  for (int i = 0; i < 7; i++)
    printf("  %-34s %7.3f ms  %6.3f ns per wave-instruction per SIMD  (%.2f x v_fma_f32)\n", names[i], ms[i],
           ms[i] * 1e6 / per_simd, ms[i] / ms[0]);

  printf("part 2: per slot of 4 MFMAs (ns per SIMD)\n");
  for (int wps = 1; wps <= 4; wps *= 2) {
    int const b = device_cus * wps;  // 4 waves per block: wps waves per SIMD
    double const slots = double(b) * 4 * kIter / simds;
    auto row = [&](char const* name, float t) { printf("  wps=%d %-30s %7.2f\n", wps, name, t * 1e6 / slots); };
    row("4 MFMA", time_ms([&] { overlap<4, 0, 0><<<b, 256>>>(d, 0.5f); }));
    row("16 FMA", time_ms([&] { overlap<0, 4, 0><<<b, 256>>>(d, 0.5f); }));
    row("4 MFMA + 16 FMA", time_ms([&] { overlap<4, 4, 0><<<b, 256>>>(d, 0.5f); }));
    row("4 tanh chains", time_ms([&] { overlap<0, 1, 1><<<b, 256>>>(d, 0.5f); }));
    row("4 MFMA + 4 tanh chains", time_ms([&] { overlap<4, 1, 1><<<b, 256>>>(d, 0.5f); }));
    row("8 tanh chains", time_ms([&] { overlap<0, 2, 1><<<b, 256>>>(d, 0.5f); }));
    row("4 MFMA + 8 tanh chains", time_ms([&] { overlap<4, 2, 1><<<b, 256>>>(d, 0.5f); }));
  }
  (void)hipFree(d);
  return 0;
}
