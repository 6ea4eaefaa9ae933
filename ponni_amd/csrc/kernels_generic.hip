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

}  // namespace

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
