// fp32 MFMA tile kernels for states up to 128 features.
#include "mfma_f32.h"

namespace ponni_hip {
hipError_t launch_mfma_f32_mt8(int num_slots, LaunchArgs const& a, hipStream_t stream) {
  return mfma_f32::launch<8>(num_slots, a, stream);
}
}  // namespace ponni_hip
