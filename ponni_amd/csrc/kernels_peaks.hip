// Measured peaks of the device the library runs on, reported by bench.py
// beside the published ones: a streaming device copy and a read-only stream
// (HBM) and register-only
// loops of the matrix instructions the kernels use, at the occupancy of the
// 16-bit FUSED kernels (one 512-thread workgroup per CU, two waves per SIMD).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>
#include <vector>

#include "plan.h"

namespace ponni_hip {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void copy_kernel(f4 const* __restrict__ src, f4* __restrict__ dst, int64_t n) {
  int64_t const stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

// One pass: each workgroup copies 256 x U consecutive 16-byte elements, all
// U loads issued before the first store.
template <int U>
__global__ __launch_bounds__(256) void copy_unrolled(f4 const* __restrict__ src, f4* __restrict__ dst, int64_t n) {
  int64_t const base = int64_t(blockIdx.x) * 256 * U + threadIdx.x;
  f4 v[U];
#pragma unroll
  for (int u = 0; u < U; u++)
    if (base + u * 256 < n) v[u] = src[base + u * 256];
#pragma unroll
  for (int u = 0; u < U; u++)
    if (base + u * 256 < n) dst[base + u * 256] = v[u];
}

// Read-only stream: each workgroup reads 256 x U consecutive 16-byte elements
// and writes nothing unless the sum takes a value zero-filled input never gives.
template <int U>
__global__ __launch_bounds__(256) void read_unrolled(f4 const* __restrict__ src, float* __restrict__ sink, int64_t n) {
  int64_t const base = int64_t(blockIdx.x) * 256 * U + threadIdx.x;
  f4 v[U];
#pragma unroll
  for (int u = 0; u < U; u++) v[u] = base + u * 256 < n ? src[base + u * 256] : f4{0.0f, 0.0f, 0.0f, 0.0f};
  float s = 0.0f;
#pragma unroll
  for (int u = 0; u < U; u++) s += v[u][0] + v[u][1] + v[u][2] + v[u][3];
  if (s == 1.0f) sink[threadIdx.x] = s;
}

// A copy shaped like c1's NARROW kernel: 256-thread workgroups, each lane 4
// consecutive columns of two input rows (two 16-byte loads) and of one output
// row (one 16-byte store), i.e. 8 bytes read and 4 written per column.
__global__ __launch_bounds__(256) void rows2to1(f4 const* __restrict__ x, f4* __restrict__ y, int64_t n4) {
  int64_t const i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n4) y[i] = x[i] + x[n4 + i];
}

// Mean kernel duration (ms) of rows2to1 over `columns` columns, from events
// each dispatch stamps itself (hipExtLaunchKernel, as ponni_forward_timed
// times the forward kernels), over `sets` input / output pairs in rotation so
// that no launch finds its data in the MALL; -1 on failure.
float small_copy_ms(int64_t columns, int sets, hipStream_t stream) {
  int64_t const n4 = columns / 4;
  size_t const set_bytes = size_t(n4) * 16 * 3;
  char* buf = nullptr;
  if (hipMalloc(&buf, set_bytes * sets) != hipSuccess) return -1.0f;
  float result = -1.0f;
  std::vector<hipEvent_t> ev(2 * size_t(sets), nullptr);
  bool ok = hipMemsetAsync(buf, 0, set_bytes * sets, stream) == hipSuccess;
  for (auto& e : ev) ok = ok && hipEventCreate(&e) == hipSuccess;
  dim3 const grid(unsigned((n4 + 255) / 256)), block(256);
  double sum = 0.0;
  for (int pass = 0; ok && pass < 2; pass++) {  // the first pass warms up
    for (int i = 0; ok && i < sets; i++) {
      f4 const* x = reinterpret_cast<f4 const*>(buf + set_bytes * i);
      f4* y = reinterpret_cast<f4*>(buf + set_bytes * i + size_t(n4) * 32);
      int64_t n = n4;
      void* args[] = {&x, &y, &n};
      ok = hipExtLaunchKernel(reinterpret_cast<void const*>(rows2to1), grid, block, args, 0, stream, ev[2 * i],
                              ev[2 * i + 1], 0) == hipSuccess;
    }
    ok = ok && hipStreamSynchronize(stream) == hipSuccess;
    sum = 0.0;
    for (int i = 0; ok && i < sets; i++) {
      float ms = 0.0f;
      ok = hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]) == hipSuccess;
      sum += ms;
    }
  }
  if (ok) result = static_cast<float>(sum / sets);
  for (auto& e : ev)
    if (e != nullptr) (void)hipEventDestroy(e);
  (void)hipFree(buf);
  return result;
}

// Eight independent accumulators per lane; `iters` rounds of 8 MFMAs.
__global__ __launch_bounds__(512) void mfma_f16_loop(float* __restrict__ out, int iters, float seed) {
  f4 acc[8];
  h8 a, b;
  for (int j = 0; j < 8; j++) {
    acc[j] = f4{seed, 0.0f, 0.0f, 0.0f};
    a[j] = static_cast<_Float16>(0.001f * (threadIdx.x + j));
    b[j] = static_cast<_Float16>(0.002f * j);
  }
  for (int i = 0; i < iters; i++)
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[j], 0, 0, 0);
  float s = 0.0f;
  for (int j = 0; j < 8; j++) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

__global__ __launch_bounds__(512) void mfma_f32_loop(float* __restrict__ out, int iters, float seed) {
  f4 acc[8];
  float const a = 0.001f * threadIdx.x, b = 0.002f;
  for (int j = 0; j < 8; j++) acc[j] = f4{seed, 0.0f, 0.0f, 0.0f};
  for (int i = 0; i < iters; i++)
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[j], 0, 0, 0);
  float s = 0.0f;
  for (int j = 0; j < 8; j++) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Median over `reps` samples (after one warm-up launch) of the time per
// launch, in ms; each sample times `per` launches back to back between two
// events, so event overhead is spread over them.
template <class Launch>
float median_ms(Launch launch, hipStream_t stream, int reps, int per) {
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    if (e0 != nullptr) (void)hipEventDestroy(e0);
    return -1.0f;
  }
  launch();
  std::vector<float> t;
  for (int r = 0; r < reps; r++) {
    float ms = 0.0f;
    (void)hipEventRecord(e0, stream);
    for (int i = 0; i < per; i++) launch();
    (void)hipEventRecord(e1, stream);
    if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) ms = -1.0f;
    t.push_back(ms / per);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  std::sort(t.begin(), t.end());
  return t[t.size() / 2];
}

}  // namespace
}  // namespace ponni_hip

extern "C" int ponni_measure_peaks(ponni_peaks* out, hipStream_t stream) {
  using namespace ponni_hip;
  if (out == nullptr) return set_error(PONNI_ERR_INVALID_ARGUMENT, "output is null");
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return set_error(PONNI_ERR_DEVICE, "no device");
  // HBM: copy 1 GiB (read 1 GiB, write 1 GiB).
  int64_t const bytes = int64_t(1) << 30;
  void *src = nullptr, *dst = nullptr;
  float* sink = nullptr;
  if (hipMalloc(&src, bytes) != hipSuccess || hipMalloc(&dst, bytes) != hipSuccess ||
      hipMalloc(&sink, sizeof(float) * size_t(cus) * 512) != hipSuccess) {
    (void)hipFree(src);
    (void)hipFree(dst);
    return set_error(PONNI_ERR_DEVICE, "out of device memory");
  }
  if (hipMemsetAsync(src, 0, bytes, stream) != hipSuccess) {
    (void)hipFree(src);
    (void)hipFree(dst);
    (void)hipFree(sink);
    return set_error(PONNI_ERR_DEVICE, "peak measurement: memset failed");
  }
  int64_t const n4 = bytes / 16;
  // The faster of a grid-stride loop over 32 workgroups per CU and a one-pass
  // grid of 4 elements per thread.
  float const stride_ms = median_ms(
      [&] {
        hipLaunchKernelGGL(copy_kernel, dim3(cus * 32), dim3(256), 0, stream, static_cast<f4 const*>(src),
                           static_cast<f4*>(dst), n4);
      },
      stream, 5, 4);
  float const pass_ms = median_ms(
      [&] {
        hipLaunchKernelGGL(copy_unrolled<4>, dim3(unsigned((n4 + 1023) / 1024)), dim3(256), 0, stream,
                           static_cast<f4 const*>(src), static_cast<f4*>(dst), n4);
      },
      stream, 5, 4);
  float const copy_ms = std::min(stride_ms > 0.0f ? stride_ms : pass_ms, pass_ms > 0.0f ? pass_ms : stride_ms);
  float const read_ms = median_ms(
      [&] {
        hipLaunchKernelGGL(read_unrolled<4>, dim3(unsigned((n4 + 1023) / 1024)), dim3(256), 0, stream,
                           static_cast<f4 const*>(src), sink, n4);
      },
      stream, 5, 4);
  // Matrix pipes: one 512-thread workgroup per CU.
  int const iters = 4096;
  float const f16_ms = median_ms(
      [&] { hipLaunchKernelGGL(mfma_f16_loop, dim3(cus), dim3(512), 0, stream, sink, iters, 1.0f); }, stream, 3, 2);
  float const f32_ms = median_ms(
      [&] { hipLaunchKernelGGL(mfma_f32_loop, dim3(cus), dim3(512), 0, stream, sink, iters, 1.0f); }, stream, 3, 2);
  hipError_t err = hipGetLastError();
  (void)hipFree(src);
  (void)hipFree(dst);
  (void)hipFree(sink);
  // c1's traffic at c1's launch shape: 1,000,000 columns, 12 MB per launch,
  // 48 sets (576 MB) in rotation.
  int64_t const small_columns = 1000000;
  float const small_ms = err == hipSuccess ? small_copy_ms(small_columns, 48, stream) : -1.0f;
  if (err == hipSuccess) err = hipGetLastError();
  if (err != hipSuccess || copy_ms <= 0.0f || read_ms <= 0.0f || f16_ms <= 0.0f || f32_ms <= 0.0f || small_ms <= 0.0f)
    return set_error(PONNI_ERR_DEVICE, std::string("peak measurement failed: ") + hipGetErrorString(err));
  double const mfmas = double(cus) * 8 * iters * 8;  // waves x rounds x MFMAs per round
  out->hbm_copy_gbps = 2.0 * double(bytes) / (copy_ms * 1e-3) / 1e9;
  out->hbm_read_gbps = double(bytes) / (read_ms * 1e-3) / 1e9;
  out->mfma_f16_tflops = mfmas * 16384.0 / (f16_ms * 1e-3) / 1e12;  // 16x16x32: 2*16*16*32 FLOP
  out->mfma_f32_tflops = mfmas * 2048.0 / (f32_ms * 1e-3) / 1e12;   // 16x16x4: 2*16*16*4 FLOP
  out->copy_12mb_us = small_ms * 1e3;
  out->hbm_copy_12mb_gbps = 12.0 * double(small_columns) / (small_ms * 1e-3) / 1e9;
  return PONNI_OK;
}
