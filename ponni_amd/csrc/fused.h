// FUSED path: per-plan generated kernels compiled with hipRTC (fused.cpp).
#pragma once

#include <string>
#include <vector>

#include "plan.h"

namespace ponni_hip {

// Packed parameter blocks up to this size are staged in LDS by the kernel.
constexpr int64_t kFusedLdsParamBytes = 64 * 1024;
// LDS of one workgroup on gfx950.
constexpr int kFusedLdsBytes = 160 * 1024;

struct FusedConfig {
  int lds_bytes = 0;          // 0: parameters stream from L2
  int vec_bytes = 0;          // LDS copy of the per-feature vectors (0: none)
  int waves = 4;              // waves per workgroup
  int waves_per_simd = 2;     // occupancy the kernel is compiled for
  bool params_in_registers = false;  // parameters loaded once per wave, kept in VGPRs
  bool saved_in_lds = false;         // Save_State slots kept in LDS, not registers
  bool persistent_loop = false;      // staged 16-bit plans: one workgroup per CU loops over tiles
  int columns_per_block = 128;
  int lds_total = 0;                 // bytes of LDS the kernel declares
};

// Widest state a FUSED kernel of this dtype keeps on chip.
int fused_max_width(int dtype);
bool fused_supports(ponni_plan_s const& p);
// Can the NARROW plan run as a generated kernel (narrow_jit.h)?
bool narrow_jit_supports(ponni_plan_s const& p);
std::string fused_kernel_name(ponni_plan_s const& p);
std::string fused_source(ponni_plan_s const& p, FusedConfig& cfg);
// Compile (or fetch from cache) the plan's kernel; needs no device.  The
// first call settles the plan's occupancy (ponni_plan_s::fused_wps).
int fused_compile(ponni_plan_s& p, std::string& key, std::vector<char>& code, std::string& error);
// Compile if needed and load the module on the current device.
int fused_prepare(ponni_plan_s& p, std::string& error);
hipError_t fused_launch(ponni_plan_s const& p, LaunchArgs const& a, hipStream_t stream);

}  // namespace ponni_hip
