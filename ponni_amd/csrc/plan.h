// Internal plan object behind the ponni_plan handle of include/ponni_hip.h.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <array>
#include <cstdint>
#include <string>
#include <vector>

#include "../../include/ponni_hip.h"
#include "program.h"

struct ponni_plan_s;

namespace ponni_hip {

// Device launch entry points, one per kernel family (kernels_*.hip).
struct LaunchArgs {
  const Op* ops;
  int32_t num_ops;
  const Step* steps;
  const void* params;
  int64_t param_count;  // packed parameter elements
  const void* x;
  int64_t ld_x;
  void* y;
  int64_t ld_y;
  int64_t batch;
  int32_t num_inputs;
  int32_t num_outputs;
  // generic path: input, output, tmp1, tmp2, then the saved-slot area
  // (unused elsewhere), and the slot row table of that area (generic_ops.h Bufs)
  void* buffers[BUF_SAVED + 1];
  int64_t buffer_ld[BUF_SAVED + 1];
  const int32_t* slot_rows;
  // Host side only (kernels ignore them): events the runtime stamps with the
  // start and end of the kernel's own dispatch (ponni_forward_timed), or null.
  hipEvent_t ev_start;
  hipEvent_t ev_stop;
};

// Launch `kernel` on `stream`; with the timing events of `a` set, through the
// runtime's extended launch, which stamps them with the dispatch's start and end.
template <typename... Args, typename F = void (*)(Args...)>
inline void launch_kernel(F kernel, dim3 grid, dim3 block, uint32_t shmem, hipStream_t stream, LaunchArgs const& a,
                          Args... args) {
  void* argv[] = {static_cast<void*>(&args)...};
  auto const fn = reinterpret_cast<void const*>(kernel);
  if (a.ev_start != nullptr || a.ev_stop != nullptr)
    (void)hipExtLaunchKernel(fn, grid, block, argv, shmem, stream, a.ev_start, a.ev_stop, 0);
  else
    (void)hipLaunchKernel(fn, grid, block, argv, shmem, stream);
}

// Kinds of packed parameter slots (plan.cpp visit_param_slots).
enum SlotKind { SLOT_VALUE = 0, SLOT_HALF = 1, SLOT_WORD = 2 };

// One parameter segment of a layer shared with a caller-owned array
// (ponni_plan_share_layer_params): element e of the segment lives at element
// (e / cols) * ld + e % cols of `ptr`, of type `dtype`.
struct SharedSegment {
  void const* ptr = nullptr;
  int32_t dtype = 0;
  int32_t on_device = 0;
  int64_t cols = 0;
  int64_t ld = 0;
};
// A packed slot that ponni_forward refreshes from a device-shared array
// before the forward kernel, and the arrays it reads (kernels_gather.hip).
struct GatherEntry {
  int64_t slot;  // packed slot of kind `kind`
  int64_t src;   // element offset in the shared array
  int32_t seg;   // index into the GatherSource table
  int32_t kind;  // SlotKind
};
struct GatherSource {
  void const* ptr;
  int32_t dtype;
  int32_t pad;
};
hipError_t launch_gather(GatherEntry const* map, int64_t count, GatherSource const* sources, void* packed,
                         int plan_dtype, hipStream_t stream);

// Fixed device scratch of ponni_forward_no_alloc (static_scratch.hip): the
// device address of this device's copy (looked up on the first call with
// `device` current; no allocation).
constexpr size_t kStaticScratchBytes = size_t(PONNI_NO_ALLOC_SCRATCH_BYTES);
hipError_t static_scratch(int device, void** out);

hipError_t launch_generic(int dtype, LaunchArgs const& args, hipStream_t stream);
// One dense op of a LAYERED plan (kernels_generic.hip layered_dense): in and
// out are the op's state buffers, params the plan's packed parameters in the
// compute type (GENERIC packing: W [n_in][n_out] at woff).
struct DenseArgs {
  const void* x;
  int64_t ldx;
  void* y;
  int64_t ldy;
  int64_t batch;
  const void* params;
  int32_t woff;
  int32_t n_in;
  int32_t n_out;
  int32_t epi_begin;
  int32_t epi_count;
  int32_t bias_first;  // the first step is a bias that seeds the sum
  const Step* steps;
};
hipError_t launch_layered_dense(int dtype, DenseArgs const& a, hipStream_t stream);
hipError_t launch_narrow(int dtype, int width_class, int num_slots, LaunchArgs const& args,
                         hipStream_t stream);
hipError_t launch_mfma(int dtype, int width_class, int num_slots, LaunchArgs const& args,
                       hipStream_t stream);
hipError_t launch_fill(void* x, int dtype, int64_t n, uint64_t seed, uint64_t tag, int dist,
                       double a, double b, hipStream_t stream);

// The plan's GENERIC twin (created on first use; owned by the plan), and the
// same with its host parameter copy brought up to date.
ponni_plan_s* generic_twin(ponni_plan_s& plan);
int set_error(int status, std::string const& message);  // ponni_last_error(); returns status
int host_twin(ponni_plan_s& plan, ponni_plan_s*& twin);

// FUSED fp32 / fp64 plans whose input width is not a multiple of 16 and
// whose input state is only ever read by dense contractions (Matvec, Dense,
// the projection of Binop_Projection_Add; through saves and loads): the
// packed-parameter offsets of those contractions.  Their input tile then
// holds feature 4s + g in lane group g, element e of input tile m, s = 4m +
// e (contraction order), so the all-padding steps of those contractions are
// skipped; the weight packing and the kernel agree on it.  Empty otherwise.
std::vector<int32_t> input_contractions(ponni_plan_s const& p);

// Width classes each register path is instantiated for.
int narrow_width_class(int max_width);      // 0 if too wide
int mfma_width_class(int dtype, int max_width);  // tiles of 16 features; 0 if too wide
constexpr int kNarrowMaxSlots = 2;     // interpreted NARROW kernels
constexpr int kNarrowJitMaxSlots = 4;  // generated NARROW kernels (one register state per slot)
constexpr int kMfmaMaxSlots = 2;

}  // namespace ponni_hip

struct ponni_plan_s {
  std::vector<ponni_layer_desc> layers;
  int32_t dtype = PONNI_F32;
  int32_t path = PONNI_PATH_GENERIC;
  int32_t width_class = 0;
  int32_t max_width = 0;
  int32_t num_slots = 0;           // get_num_saved_states()
  bool external = false;           // holds PONNI_LAYER_EXTERNAL layers
  int32_t num_fused_blocks = 0;
  int32_t tmp_features[2] = {0, 0};
  std::vector<int32_t> saved_features;  // per slot, num_slots entries
  // Row of each slot in the saved-state area (max(num_slots, 1) entries)
  // and the area's height, the sum of the slots' widths.
  std::vector<int32_t> slot_rows;
  int32_t saved_total = 0;

  // Host master copy of every layer's parameters (exact in double).
  std::vector<std::vector<double>> params;

  // Lowered program; offsets into the packed parameter buffer of `path`.
  std::vector<ponni_hip::Op> ops;
  std::vector<ponni_hip::Step> steps;
  std::vector<int64_t> layer_param_offset;  // per layer, in packed elements
  int64_t packed_elements = 0;

  // Device state.
  bool device_dirty = true;
  int device = -1;
  ponni_hip::Op* d_ops = nullptr;
  ponni_hip::Step* d_steps = nullptr;
  int32_t* d_slot_rows = nullptr;
  size_t d_ops_count = 0, d_steps_count = 0;  // capacities of d_ops / d_steps
  void* d_params = nullptr;
  size_t d_params_bytes = 0;
  void* d_scratch[3] = {};  // tmp1, tmp2, the saved-slot area
  int64_t capacity = 0;

  // GENERIC twin of this plan for ponni_plan_device_model (created on first
  // use), and the parameter version it last uploaded.
  ponni_plan_s* device_twin = nullptr;
  uint64_t params_version = 1;
  uint64_t twin_version = 0;
  // Host execution (ponni_forward_host, ponni_plan_host_model): the twin's
  // packed parameters in the compute type, and the version they were made at.
  std::vector<double> host_params_f64;
  std::vector<float> host_params_f32;
  uint64_t host_version = 0;
  // NARROW plans run a generated kernel (narrow_jit.h) unless JIT is off.
  bool narrow_jit = false;
  // FUSED path (and generated NARROW): the plan's generated kernel (compiled on first forward).
  hipFunction_t fused_fn = nullptr;
  int fused_blocks_per_cu = 1;
  int fused_cus = 0;              // compute units of the plan's device
  bool fused_persistent = false;  // grid sized to the resident workgroups
  int fused_columns_per_block = 128;
  int fused_waves = 4;  // waves per workgroup
  int fused_wps = 0;    // waves per SIMD the kernel is compiled for (0: not settled yet)

  // Parameter segments shared with caller-owned arrays (two per layer at
  // most), and the gather map that refreshes the device-shared ones.
  std::vector<std::array<ponni_hip::SharedSegment, 2>> shared;
  int num_shared_device = 0;
  int num_shared_host = 0;
  ponni_hip::GatherEntry* d_gather = nullptr;
  ponni_hip::GatherSource* d_gather_src = nullptr;
  int64_t gather_count = 0;
};
