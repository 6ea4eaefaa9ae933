// Width-class dispatch of the MFMA kernel families.
#include "plan.h"

namespace ponni_hip {

hipError_t launch_mfma_f32_mt2(int num_slots, LaunchArgs const& a, hipStream_t stream);
hipError_t launch_mfma_f32_mt4(int num_slots, LaunchArgs const& a, hipStream_t stream);
hipError_t launch_mfma_f32_mt8(int num_slots, LaunchArgs const& a, hipStream_t stream);

int mfma_width_class(int dtype, int max_width) {
  if (dtype != PONNI_F32) return 0;
  int const tiles = (max_width + 15) / 16;
  if (tiles <= 2) return 2;
  if (tiles <= 4) return 4;
  if (tiles <= 8) return 8;
  return 0;
}

hipError_t launch_mfma(int dtype, int width_class, int num_slots, LaunchArgs const& a, hipStream_t stream) {
  (void)dtype;
  switch (width_class) {
    case 2: return launch_mfma_f32_mt2(num_slots, a, stream);
    case 4: return launch_mfma_f32_mt4(num_slots, a, stream);
    default: return launch_mfma_f32_mt8(num_slots, a, stream);
  }
}

}  // namespace ponni_hip
