// LDS read rate next to v_mfma_f32_16x16x32_f16 on gfx950 (not a test:
// built and run by hand, its output summarized with the command that made
// it).  The 16-bit FUSED kernels read each 1 KB A fragment (16 output
// features x 32 inputs) from LDS once per wave and use it for NT MFMAs, one
// per 16-column tile the wave owns; this measures what that costs the matrix
// pipe for NT = 1..4, with 8 waves per CU (two per SIMD, the kernels'
// occupancy):
//   - "A in registers": R MFMAs per iteration on a fragment held in VGPRs;
//   - "ds_read + R MFMA": a fragment read from LDS, then R MFMAs on it, the
//     read waited for just before its MFMAs;
//   - "... read ahead": the next iteration's fragment requested before this
//     iteration's MFMAs, so the read has R MFMAs to arrive in.
// Every kernel writes one float per thread into a buffer sized for the
// launch; the values are discarded.
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       tests/perf/lds_mfma_rates.hip -o /tmp/lds_mfma_rates && /tmp/lds_mfma_rates
#include <hip/hip_runtime.h>

#include <cstdio>

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
constexpr int kIter = 65536;
constexpr int kFrags = 32;  // 32 KB of fragments, as one LDS slot of the kernels

// MODE 0: A from registers; 1: read, wait, R MFMAs; 2: read one iteration ahead.
template <int R, int MODE>
__global__ __launch_bounds__(512) void probe(float* out, float seed) {
  __shared__ h8 buf[kFrags * 64];
  int const lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < kFrags * 64; i += blockDim.x)
    for (int j = 0; j < 8; j++) buf[i][j] = static_cast<_Float16>(0.001f * (i + j) * seed);
  __syncthreads();
  f4 acc[8];
  for (int j = 0; j < 8; j++) acc[j] = f4{seed, 0, 0, 0};
  h8 b;
  for (int j = 0; j < 8; j++) b[j] = static_cast<_Float16>(0.01f * (lane + j));
  h8 next = buf[(w % kFrags) * 64 + lane];
  for (int i = 0; i < kIter; i += 4) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
      h8 a;
      if constexpr (MODE == 0) {
        a = b;
      } else if constexpr (MODE == 1) {
        a = buf[((i + u + w) % kFrags) * 64 + lane];
      } else {
        a = next;
        next = buf[((i + u + 1 + w) % kFrags) * 64 + lane];
        __builtin_amdgcn_sched_barrier(0);  // keep the request above the MFMAs
      }
#pragma unroll
      for (int r = 0; r < R; r++)
        acc[(u * R + r) % 8] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[(u * R + r) % 8], 0, 0, 0);
    }
  }
  float s = static_cast<float>(next[0]);
  for (int j = 0; j < 8; j++) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
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
  int cus = 0;
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0);
  float* d = nullptr;
  if (hipMalloc(&d, sizeof(float) * cus * 512) != hipSuccess) return 1;
  // One 512-thread workgroup per CU: 8 waves, two per SIMD.
  auto row = [&](char const* name, int R, bool lds, float ms) {
    double const mfma_per_simd = double(8) * kIter * R / 4;
    double const ns = ms * 1e6 / mfma_per_simd;
    double const lds_bytes_per_ns = lds ? double(8) * kIter * 1024 / (ms * 1e6) : 0.0;  // per CU
    printf("  %-34s R=%d  %8.3f ms  %6.2f ns per MFMA per SIMD  LDS %6.1f B/ns per CU\n", name, R, ms, ns,
           lds_bytes_per_ns);
  };
  printf("8 waves per CU, %d CUs; MFMA = v_mfma_f32_16x16x32_f16\n", cus);
  row("A in registers", 1, false, time_ms([&] { probe<1, 0><<<cus, 512>>>(d, 1.0f); }));
  row("A in registers", 2, false, time_ms([&] { probe<2, 0><<<cus, 512>>>(d, 1.0f); }));
  row("A in registers", 4, false, time_ms([&] { probe<4, 0><<<cus, 512>>>(d, 1.0f); }));
  row("ds_read_b128, then R MFMA", 1, true, time_ms([&] { probe<1, 1><<<cus, 512>>>(d, 1.0f); }));
  row("ds_read_b128, then R MFMA", 2, true, time_ms([&] { probe<2, 1><<<cus, 512>>>(d, 1.0f); }));
  row("ds_read_b128, then R MFMA", 3, true, time_ms([&] { probe<3, 1><<<cus, 512>>>(d, 1.0f); }));
  row("ds_read_b128, then R MFMA", 4, true, time_ms([&] { probe<4, 1><<<cus, 512>>>(d, 1.0f); }));
  row("ds_read_b128 read ahead, R MFMA", 1, true, time_ms([&] { probe<1, 2><<<cus, 512>>>(d, 1.0f); }));
  row("ds_read_b128 read ahead, R MFMA", 2, true, time_ms([&] { probe<2, 2><<<cus, 512>>>(d, 1.0f); }));
  row("ds_read_b128 read ahead, R MFMA", 3, true, time_ms([&] { probe<3, 2><<<cus, 512>>>(d, 1.0f); }));
  (void)hipFree(d);
  return 0;
}
