// Counter-based synthetic data on the device (bench and test inputs).
// u64(i) = splitmix64(key + i) with key = splitmix64(seed ^ splitmix64(tag));
// uniform = a + (b - a) * (top 24 bits * 2^-24), evaluated as one fma in
// double so the host generator reproduces it bit for bit; normal = Box-Muller
// on the uniforms of indices 2i and 2i+1.
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "plan.h"

namespace ponni_hip {
namespace {

__device__ inline uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

template <class S> __device__ inline S cast_out(float v) { return static_cast<S>(v); }
template <> __device__ inline __half cast_out<__half>(float v) { return __float2half_rn(v); }
template <> __device__ inline __hip_bfloat16 cast_out<__hip_bfloat16>(float v) { return __float2bfloat16(v); }

template <class S>
__global__ void fill_kernel(S* __restrict__ x, int64_t n, uint64_t key, int dist, double a, double b) {
  int64_t const stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    double v;
    if (dist == 0) {
      double const u = double(splitmix64(key + uint64_t(i)) >> 40) * (1.0 / 16777216.0);
      v = fma(b - a, u, a);
    } else {
      double const u1 = double((splitmix64(key + 2 * uint64_t(i)) >> 40) + 1) * (1.0 / 16777216.0);
      double const u2 = double(splitmix64(key + 2 * uint64_t(i) + 1) >> 40) * (1.0 / 16777216.0);
      v = a + b * (sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
    }
    x[i] = cast_out<S>(static_cast<float>(v));
  }
}

template <> __global__ void fill_kernel<double>(double* __restrict__ x, int64_t n, uint64_t key, int dist, double a,
                                                double b) {
  int64_t const stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    if (dist == 0) {
      double const u = double(splitmix64(key + uint64_t(i)) >> 40) * (1.0 / 16777216.0);
      x[i] = fma(b - a, u, a);
    } else {
      double const u1 = double((splitmix64(key + 2 * uint64_t(i)) >> 40) + 1) * (1.0 / 16777216.0);
      double const u2 = double(splitmix64(key + 2 * uint64_t(i) + 1) >> 40) * (1.0 / 16777216.0);
      x[i] = a + b * (sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
    }
  }
}

uint64_t host_splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

}  // namespace

hipError_t launch_fill(void* x, int dtype, int64_t n, uint64_t seed, uint64_t tag, int dist, double a, double b,
                       hipStream_t stream) {
  uint64_t const key = host_splitmix64(seed ^ host_splitmix64(tag));
  int64_t const blocks64 = (n + 255) / 256;
  dim3 const grid(static_cast<unsigned>(blocks64 < 65536 ? blocks64 : 65536));
  dim3 const block(256);
  switch (dtype) {
    case PONNI_F64:
      hipLaunchKernelGGL(fill_kernel<double>, grid, block, 0, stream, static_cast<double*>(x), n, key, dist, a, b);
      break;
    case PONNI_F16:
      hipLaunchKernelGGL(fill_kernel<__half>, grid, block, 0, stream, static_cast<__half*>(x), n, key, dist, a, b);
      break;
    case PONNI_BF16:
      hipLaunchKernelGGL(fill_kernel<__hip_bfloat16>, grid, block, 0, stream, static_cast<__hip_bfloat16*>(x), n,
                         key, dist, a, b);
      break;
    default:
      hipLaunchKernelGGL(fill_kernel<float>, grid, block, 0, stream, static_cast<float*>(x), n, key, dist, a, b);
      break;
  }
  return hipGetLastError();
}

}  // namespace ponni_hip
