// Refresh of shared parameters: before a forward pass, every packed slot
// whose parameter lives in a caller-owned device array (a layer View shared
// with the model, ponni_plan_share_layer_params) is re-read from that array
// in stream order and converted to the packed form, so writes the caller
// made to the array before the forward are what the forward kernel sees.
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "plan.h"

namespace ponni_hip {
namespace {

__device__ inline double load_element(void const* p, int dtype, int64_t i) {
  switch (dtype) {
    case PONNI_F64: return static_cast<double const*>(p)[i];
    case PONNI_F16: return static_cast<double>(__half2float(static_cast<__half const*>(p)[i]));
    case PONNI_BF16: return static_cast<double>(__bfloat162float(static_cast<__hip_bfloat16 const*>(p)[i]));
    default: return static_cast<double>(static_cast<float const*>(p)[i]);
  }
}

// The value as the plan's parameter type holds it (round to nearest even).
__device__ inline float round_to_type(float v, int dtype) {
  if (dtype == PONNI_F16) return __half2float(__float2half(v));
  if (dtype == PONNI_BF16) return __bfloat162float(__float2bfloat16(v));
  return v;
}

__global__ __launch_bounds__(256) void gather_params(GatherEntry const* __restrict__ map, int64_t count,
                                                     GatherSource const* __restrict__ sources, void* packed,
                                                     int plan_dtype) {
  int64_t const i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= count) return;
  GatherEntry const e = map[i];
  GatherSource const s = sources[e.seg];
  double const v = load_element(s.ptr, s.dtype, e.src);
  if (e.kind == SLOT_HALF) {
    unsigned short const bits = plan_dtype == PONNI_F16 ? __half_as_ushort(__float2half(static_cast<float>(v)))
                                                        : __bfloat16_as_ushort(__float2bfloat16(static_cast<float>(v)));
    static_cast<unsigned short*>(packed)[e.slot] = bits;
  } else if (plan_dtype == PONNI_F64) {
    static_cast<double*>(packed)[e.slot] = v;
  } else {
    static_cast<float*>(packed)[e.slot] = round_to_type(static_cast<float>(v), plan_dtype);
  }
}

}  // namespace

hipError_t launch_gather(GatherEntry const* map, int64_t count, GatherSource const* sources, void* packed,
                         int plan_dtype, hipStream_t stream) {
  if (count <= 0) return hipSuccess;
  dim3 const grid(static_cast<unsigned>((count + 255) / 256));
  hipLaunchKernelGGL(gather_params, grid, dim3(256), 0, stream, map, count, sources, packed, plan_dtype);
  return hipGetLastError();
}

}  // namespace ponni_hip
