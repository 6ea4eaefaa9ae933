/*
 * ponni_hip.h -- C ABI of libponni_hip.so, the MI355X (gfx950) implementation
 * of PONNI's batched forward pass.
 *
 * The reference has no FFI: its operator API is the compile-time C++ layer
 * contract plus the Inference model object.  Every entry point below replaces
 * one piece of that contract; the reference file:line it stands in for is
 * cited on each declaration (paths are relative to the reference root).  The
 * header-only C++ facade in ponni_amd/include/ponni.h rebuilds the reference's
 * C++ API (create_inference_model, the layer templates, Inference, PonniFile)
 * on top of these functions.
 *
 * Conventions
 *   - Status: every int-returning call returns PONNI_OK (0) or a nonzero
 *     ponni_status; ponni_last_error() then holds a thread-local message.
 *   - Layout: activations are feature-major [features, batch]; element (f, b)
 *     of a buffer with row stride ld lives at base + f*ld + b (LayoutRight).
 *   - Ownership: callers own input and output buffers; a plan owns only its
 *     device weights and retained scratch.
 *   - Streams: ponni_forward is asynchronous on the caller's stream and never
 *     synchronizes (a null stream means the default stream).
 */
#ifndef PONNI_HIP_H
#define PONNI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifndef HIP_INCLUDE_HIP_HIP_RUNTIME_API_H
typedef struct ihipStream_t* hipStream_t;
typedef struct ihipEvent_t* hipEvent_t;
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define PONNI_ABI_VERSION 1

typedef enum ponni_status {
  PONNI_OK = 0,
  PONNI_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad enum, negative size  */
  PONNI_ERR_INVALID_MODEL = 2,    /* layer chain fails Inference::validate  */
  PONNI_ERR_SHAPE = 3,            /* batch == 0 or extents do not match      */
  PONNI_ERR_UNSUPPORTED = 4,      /* forced kernel path cannot run the model */
  PONNI_ERR_DEVICE = 5,           /* HIP runtime error                      */
  PONNI_ERR_IO = 6                /* .ponni file rejected                    */
} ponni_status;

/* Element type of activations (and of the arithmetic that produces them). */
typedef enum ponni_dtype {
  PONNI_F32 = 1,
  PONNI_F64 = 2,
  PONNI_F16 = 3,  /* fp16 operands, fp32 accumulation */
  PONNI_BF16 = 4  /* bf16 operands, fp32 accumulation */
} ponni_dtype;

/* Built-in layer templates, src/ponni.h:27-48 of the reference. */
typedef enum ponni_layer_kind {
  PONNI_LAYER_MATVEC = 1,        /* layers/ponni_Matvec.h: W [n_in, n_out]          */
  PONNI_LAYER_BIAS = 2,          /* layers/ponni_Bias.h: b [n]                       */
  PONNI_LAYER_RELU = 3,          /* layers/ponni_Relu.h                              */
  PONNI_LAYER_LEAKY_RELU = 4,    /* layers/ponni_LeakyRelu.h: attr[0] negative_slope */
  PONNI_LAYER_ELU = 5,           /* layers/ponni_Elu.h: attr[0] alpha                */
  PONNI_LAYER_SELU = 6,          /* layers/ponni_Selu.h                              */
  PONNI_LAYER_GELU = 7,          /* layers/ponni_Gelu.h: flags bit0 = approximate    */
  PONNI_LAYER_SILU = 8,          /* layers/ponni_Silu.h                              */
  PONNI_LAYER_SIGMOID = 9,       /* layers/ponni_Sigmoid.h                           */
  PONNI_LAYER_TANH = 10,         /* layers/ponni_Tanh.h                              */
  PONNI_LAYER_SOFTPLUS = 11,     /* layers/ponni_Softplus.h: attr[0] beta            */
  PONNI_LAYER_HARD_SIGMOID = 12, /* layers/ponni_HardSigmoid.h: attr[0] alpha, [1] beta */
  PONNI_LAYER_HARD_SWISH = 13,   /* layers/ponni_HardSwish.h                         */
  PONNI_LAYER_MISH = 14,         /* layers/ponni_Mish.h                              */
  PONNI_LAYER_SOFTMAX = 20,      /* layers/ponni_Softmax.h (barrier)                 */
  PONNI_LAYER_LOG_SOFTMAX = 21,  /* layers/ponni_LogSoftmax.h (barrier)              */
  PONNI_LAYER_LAYER_NORM = 22,   /* layers/ponni_LayerNorm.h: gamma[n], beta[n]; attr[0] epsilon */
  PONNI_LAYER_MIN_MAX_NORM = 23, /* layers/ponni_MinMaxNorm.h: attr out_min, out_max, epsilon */
  PONNI_LAYER_SAVE_STATE = 30,   /* layers/ponni_Save_State.h: slot = ISAVE          */
  PONNI_LAYER_BINOP_ADD = 31,    /* layers/ponni_Binop_Add.h: slot = ISAVE           */
  PONNI_LAYER_BINOP_CONCATENATE = 32, /* layers/ponni_Binop_Concatenate.h: slot; n_in = N1,
                                         n_out = N1 + N2; flags bit0 = after         */
  PONNI_LAYER_BINOP_PROJECTION_ADD = 33, /* layers/ponni_Binop_Projection_Add.h: slot;
                                           n_aux = NSAVE; W [NSAVE, n_in], bias [n_in] */

  /* Operations of generated graphs (the canonical IR of kokkos_nn/ir.py as the
   * emitter lowers it, kokkos_nn/emitter.py:693-941).  They have no layer
   * template; ponni_amd/graph.py linearizes a graph into a chain that uses
   * them together with the kinds above. */
  PONNI_LAYER_DENSE = 40,        /* emitter.py:693-734: W [n_out, n_in] row-major, then
                                    bias [n_out] when flags bit0; sum = bias, += W x   */
  PONNI_LAYER_LOAD_STATE = 41,   /* state = saved[slot]; n_out = that slot's width      */
  PONNI_LAYER_BINARY = 42,       /* emitter.py:735-741: state = op(a, b) of the state and
                                    saved[slot]; attr[0] = ponni_binary_op; flags bit0 =
                                    saved operand on the left; n_aux = saved width; each
                                    operand has 1 or n_out features (scalar broadcast) */
  PONNI_LAYER_REDUCE = 43,       /* emitter.py:475-547: n_in features -> 1;
                                    attr[0] = ponni_reduce_op                           */
  PONNI_LAYER_UNARY = 44,        /* emitter.py:218-258: pointwise; attr[0] = ponni_unary_op,
                                    attr[1] alpha, attr[2] gamma                       */
  PONNI_LAYER_CONST_BINARY = 45, /* pointwise op(state, c) with a constant c [n_in];
                                    attr[0] = ponni_binary_op; flags bit0 = c on the left */
  PONNI_LAYER_SELECT = 46,       /* interpreter.py:178-183 Where / CompareSelect: cond != 0 ?
                                    a : b over n_out features.  Each operand comes from
                                    the state, a saved slot or a constant (flags: 2 bits
                                    per operand, PONNI_SELECT_*); the first slot operand
                                    is saved[slot], the second saved[attr[1]]; a one-
                                    feature operand broadcasts (flags bits 6-8); constant
                                    a, then constant b, are the layer's parameters
                                    [n_out] each.  The condition is never a constant. */

  /* A layer the library does not implement: a user layer of the C++ facade
   * under the reference's plugin contract (ponni_LayerTraits.h:10-61; its
   * device functions compute_output / apply_fused / compute_all_outputs run
   * in the facade's per-sample kernel).  attr[0] = the caller's index for it;
   * flags: PONNI_FLAG_EXT_* below; slot = ISAVE when it saves or reads a
   * saved state.  A plan holding one is always GENERIC, is evaluated only
   * through ponni_plan_device_model with the caller's callback
   * (ponni_amd/include/ponni/device.h), and ponni_forward rejects it. */
  PONNI_LAYER_EXTERNAL = 50
} ponni_layer_kind;

/* Element-wise binary operations of PONNI_LAYER_BINARY / _CONST_BINARY. */
typedef enum ponni_binary_op {
  PONNI_BINARY_ADD = 0,
  PONNI_BINARY_SUB = 1,
  PONNI_BINARY_MUL = 2,
  PONNI_BINARY_DIV = 3,
  PONNI_BINARY_MIN = 4, /* a < b ? a : b */
  PONNI_BINARY_MAX = 5, /* a > b ? a : b */
  PONNI_BINARY_POW = 6,
  /* comparisons and logic give 1 or 0 (interpreter.py:132-162; a boolean is
   * 1 / 0 in the state, anything nonzero is true) */
  PONNI_BINARY_EQUAL = 7,
  PONNI_BINARY_GREATER = 8,
  PONNI_BINARY_GREATER_EQUAL = 9,
  PONNI_BINARY_LESS = 10,
  PONNI_BINARY_LESS_EQUAL = 11,
  PONNI_BINARY_AND = 12,
  PONNI_BINARY_OR = 13,
  PONNI_BINARY_XOR = 14,
  PONNI_BINARY_PRELU = 15 /* a >= 0 ? a : a * b (interpreter.py:164-165) */
} ponni_binary_op;

/* Feature reductions of PONNI_LAYER_REDUCE (emitter.py:475-512). */
typedef enum ponni_reduce_op {
  PONNI_REDUCE_SUM = 0,
  PONNI_REDUCE_MEAN = 1,
  PONNI_REDUCE_MAX = 2,
  PONNI_REDUCE_MIN = 3,
  PONNI_REDUCE_L1 = 4,
  PONNI_REDUCE_L2 = 5,
  PONNI_REDUCE_SUM_SQUARE = 6,
  PONNI_REDUCE_LOG_SUM = 7,
  PONNI_REDUCE_LOG_SUM_EXP = 8,
  PONNI_REDUCE_PROD = 9
} ponni_reduce_op;

/* Unary operations of PONNI_LAYER_UNARY without a layer template
 * (emitter.py:218-258). */
typedef enum ponni_unary_op {
  PONNI_UNARY_ABS = 0,
  PONNI_UNARY_NEG = 1,
  PONNI_UNARY_EXP = 2,
  PONNI_UNARY_LOG = 3,
  PONNI_UNARY_SQRT = 4,
  PONNI_UNARY_RECIPROCAL = 5,
  PONNI_UNARY_SOFTSIGN = 6,
  PONNI_UNARY_CELU = 7,             /* attr[1] alpha */
  PONNI_UNARY_THRESHOLDED_RELU = 8, /* attr[1] alpha */
  PONNI_UNARY_ERF = 9,
  PONNI_UNARY_SELU = 10,            /* attr[1] alpha, attr[2] gamma: gamma * (x > 0 ? x : alpha*(e^x - 1)) */
  PONNI_UNARY_ACOS = 11,
  PONNI_UNARY_ACOSH = 12,
  PONNI_UNARY_ASIN = 13,
  PONNI_UNARY_ASINH = 14,
  PONNI_UNARY_ATAN = 15,
  PONNI_UNARY_ATANH = 16,
  PONNI_UNARY_CEIL = 17,
  PONNI_UNARY_COS = 18,
  PONNI_UNARY_COSH = 19,
  PONNI_UNARY_FLOOR = 20,
  PONNI_UNARY_SIN = 21,
  PONNI_UNARY_SINH = 22,
  PONNI_UNARY_TAN = 23,
  PONNI_UNARY_ROUND = 24,           /* to nearest, ties to even (numpy round) */
  PONNI_UNARY_SIGN = 25,            /* -1, 0, 1; NaN stays NaN */
  PONNI_UNARY_IS_NAN = 26,          /* 1 / 0 */
  PONNI_UNARY_IS_INF = 27,          /* 1 / 0; attr[1] detect_negative, attr[2] detect_positive */
  PONNI_UNARY_NOT = 28,             /* x == 0 ? 1 : 0 */
  PONNI_UNARY_NONZERO = 29          /* Cast to bool: x != 0 ? 1 : 0 */
} ponni_unary_op;

/* Operand sources of PONNI_LAYER_SELECT (2 bits each in flags: cond bits 0-1,
 * a bits 2-3, b bits 4-5), and its one-feature (broadcast) operand flags. */
#define PONNI_SELECT_STATE 0
#define PONNI_SELECT_SLOT 1
#define PONNI_SELECT_CONST 2
#define PONNI_SELECT_COND_SCALAR 64
#define PONNI_SELECT_A_SCALAR 128
#define PONNI_SELECT_B_SCALAR 256

#define PONNI_FLAG_DENSE_BIAS 1 /* PONNI_LAYER_DENSE carries a bias     */
#define PONNI_FLAG_SAVED_LEFT 1 /* PONNI_LAYER_BINARY: saved[slot] op state */
#define PONNI_FLAG_CONST_LEFT 1 /* PONNI_LAYER_CONST_BINARY: c op state  */
#define PONNI_FLAG_EXT_SAVE 1     /* PONNI_LAYER_EXTERNAL: output goes to saved[slot] (save = true) */
#define PONNI_FLAG_EXT_BINOP 2    /* PONNI_LAYER_EXTERNAL: also reads saved[slot] (binop = true)   */
#define PONNI_FLAG_EXT_IN_PLACE 4 /* PONNI_LAYER_EXTERNAL: overwrite_input = true                 */

/* One layer of the tuple handed to create_inference_model
 * (src/ponni_create_model.h:40-65).  Widths are the runtime extents the
 * reference reads from each layer's Views (e.g. ponni_Matvec.h:62-65). */
typedef struct ponni_layer_desc {
  int32_t kind;    /* ponni_layer_kind                                      */
  int32_t n_in;    /* get_num_inputs()                                      */
  int32_t n_out;   /* get_num_outputs()                                     */
  int32_t slot;    /* ISAVE of Save_State / Binop_*; ignored otherwise      */
  int32_t n_aux;   /* NSAVE of Binop_Projection_Add; ignored otherwise      */
  int32_t flags;   /* PONNI_FLAG_*                                          */
  double attr[4];  /* scalar configuration (slope, alpha, beta, epsilon...) */
} ponni_layer_desc;

#define PONNI_FLAG_GELU_APPROXIMATE 1 /* Gelu(n, approximate = true)      */
#define PONNI_FLAG_CONCAT_AFTER 1     /* Binop_Concatenate(.., after=true) */

/* Kernel families a plan can run on. */
typedef enum ponni_path {
  PONNI_PATH_AUTO = 0,    /* pick the fastest path that supports the model          */
  PONNI_PATH_GENERIC = 1, /* one sample per lane, states in HBM scratch (any model) */
  PONNI_PATH_NARROW = 2,  /* one sample per lane, states in registers (width <= 16) */
  PONNI_PATH_MFMA = 3,    /* 16x16 MFMA tiles, states in registers (width <= 128)   */
  PONNI_PATH_FUSED = 4,   /* MFMA tiles in a kernel generated for this plan and
                             compiled with hipRTC on first use (16-bit width
                             <= 1024, fp32 <= 512, fp64 <= 256)                     */
  PONNI_PATH_LAYERED = 5  /* the GENERIC op list with every dense block run over the
                             whole batch as an MFMA contraction (states in HBM
                             scratch; any width)                                    */
} ponni_path;

typedef struct ponni_plan_s* ponni_plan;

/* Facts about a compiled plan; mirrors the scratch-planning queries of
 * src/ponni_Inference.h:92-122, :180, :204-223 and :75-85. */
typedef struct ponni_plan_info {
  int32_t path;              /* ponni_path actually selected                      */
  int32_t dtype;             /* ponni_dtype                                       */
  int32_t num_layers;
  int32_t num_inputs;        /* first layer get_num_inputs()                      */
  int32_t num_outputs;       /* last layer get_num_outputs()                      */
  int32_t num_fused_dense_blocks;  /* get_num_fused_dense_blocks()                */
  int32_t num_saved_states;  /* get_num_saved_states()                            */
  int32_t tmp1_features;     /* get_planned_temporary_size<0>()                   */
  int32_t tmp2_features;     /* get_planned_temporary_size<1>()                   */
  int32_t saved_features[8]; /* get_saved_state_size<i>() for slots 0..7 (any
                              slot: ponni_plan_saved_state_size)              */
  int64_t num_parameters;    /* all layer parameters, trainable or not           */
  int64_t internal_state_capacity; /* internal_state_capacity()                   */
  int32_t max_width;         /* widest state anywhere in the chain                */
  int32_t width_class;       /* register tile width chosen by NARROW / MFMA       */
} ponni_plan_info;

/* --- library ------------------------------------------------------------ */

/* Thread-local text of the last failure on this thread ("" if none). */
const char* ponni_last_error(void);

/* PONNI_ABI_VERSION of the loaded library. */
int ponni_abi_version(void);

/* --- plans (the Inference object) ---------------------------------------- */

/* Validate a layer chain and build a plan; replaces detail::create_model +
 * Inference(TUPLE) + Inference::validate (ponni_create_model.h:21-34,
 * ponni_Inference.h:159-162, :719-737).  Host-only: touches no device.  Each
 * layer's parameters start at zero until ponni_plan_set_layer_params. */
int ponni_plan_create(const ponni_layer_desc* layers, int32_t num_layers,
                      int32_t dtype, int32_t path, ponni_plan* out_plan);

/* Release a plan, its device weights and scratch (Inference::~Inference). */
void ponni_plan_destroy(ponni_plan plan);

/* Describe the plan (see ponni_plan_info). */
int ponni_plan_get_info(ponni_plan plan, ponni_plan_info* info);

/* Number of parameter values layer `layer` carries, trainable or not:
 * Matvec n_in*n_out, Bias n, LayerNorm 2n (gamma then beta),
 * Projection_Add NSAVE*n_in + n_in (W then bias), Dense n_out*n_in (+ n_out
 * with a bias), Const_Binary n_in, others 0. */
int64_t ponni_plan_layer_param_count(ponni_plan plan, int32_t layer);

/* get_saved_state_size<slot>() (ponni_Inference.h:204-223) for any slot
 * index: the widest state any Save_State<slot> stores, 0 for an unused slot
 * below get_num_saved_states(); -1 with an error for a negative slot or one
 * at or beyond get_num_saved_states(). */
int32_t ponni_plan_saved_state_size(ponni_plan plan, int32_t slot);

/* Copy one layer's parameters from host memory, in the layer's own order
 * (Matvec W [n_in, n_out] row-major; LayerNorm gamma then beta;
 * Projection_Add W [NSAVE, n_in] then bias).  `values` is float for F32,
 * F16 and BF16 plans and double for F64 plans.  Replaces the layer Views
 * held by each template (e.g. ponni_Matvec.h:29-51) and their
 * set_trainable_parameters (ponni_Matvec.h:103-109).  Re-packs the device
 * copy; synchronous with respect to the host. */
int ponni_plan_set_layer_params(ponni_plan plan, int32_t layer,
                                const void* values, int64_t count);

/* Share one parameter segment of layer `layer` with a caller-owned array
 * instead of holding a copy: the rebind rule of src/ponni_create_model.h:10-18,
 * where a layer whose Views already live in the model's memory space is
 * shared with the model, so writes through the caller's View reach later
 * forward passes (unit/core/test_core_unit.cpp:516-546).  Segment 0 is the
 * layer's first View (Matvec / Dense / projection weights, Bias or constant
 * vector, LayerNorm gamma), segment 1 its second (LayerNorm beta, projection
 * or Dense bias).  The array holds the segment in the layer's own order as
 * [rows, cols] with row stride ld (elements; rows * cols = the segment's
 * parameter count), elements of `dtype` (PONNI_F32 / F64 / F16 / BF16), in
 * device memory (on_device = 1) or host memory (0).
 *   - Device arrays: each ponni_forward / ponni_forward_no_alloc /
 *     ponni_forward_timed first re-reads them on its stream (one small gather
 *     kernel into the plan's kernel layout), so a write the caller ordered
 *     before the forward on that stream is seen.
 *   - Host arrays: read at each forward call (a changed value re-uploads).
 *   - ponni_plan_get_layer_params reads the arrays; ponni_plan_set_layer_params
 *     writes into them (the reference deep-copies into the shared View).
 *   - ponni_plan_device_model / ponni_plan_host_model describe the values
 *     read at that call.
 * The array must outlive the sharing.  values = NULL ends the sharing (the
 * plan keeps the array's current contents).  Reads the array once now. */
int ponni_plan_share_layer_params(ponni_plan plan, int32_t layer, int32_t segment,
                                  const void* values, int32_t dtype, int64_t rows,
                                  int64_t cols, int64_t ld, int32_t on_device);

/* Read one layer's parameters back into host memory (same order and type). */
int ponni_plan_get_layer_params(ponni_plan plan, int32_t layer,
                                void* values, int64_t count);

/* Reallocate batch-dependent scratch to exactly `batch` columns;
 * Inference::reallocate_internal_state (ponni_Inference.h:169-176).
 * Synchronizes the device first, as the reference fences. */
int ponni_plan_reallocate_internal_state(ponni_plan plan, int64_t batch);

/* Batched forward pass: y[n_out, batch] = model(x[n_in, batch]).  Replaces
 * Inference::forward_batch_parallel(input, output) (ponni_Inference.h:352-389)
 * and the generated infer_batch (kokkos_nn/emitter.py:1537-1550, :1903-1927).
 * x and y are device pointers of the plan's dtype with row strides ld_in and
 * ld_out (>= batch).  Grows scratch on demand (ponni_Inference.h:197-199).
 * Asynchronous on `stream`; returns PONNI_ERR_SHAPE for batch <= 0, where the
 * reference aborts (ponni_Inference.h:366). */
int ponni_forward(ponni_plan plan, const void* x, int64_t ld_in, void* y,
                  int64_t ld_out, int64_t batch, hipStream_t stream);

/* ponni_forward for callers that cannot allocate device memory: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * It has no counterpart in the reference.  It calls no hipMalloc, hipFree or
 * other allocating routine: a GENERIC plan's state buffers (tmp1, tmp2 and the
 * saved slots, [features, batch] each) are carved from one fixed device array
 * of PONNI_NO_ALLOC_SCRATCH_BYTES per GPU, which every GPU the library runs on
 * holds from the first call on it until the process ends; the other paths
 * keep their states on chip and need none.  Nothing in the array has to
 * start at zero (every state is written before it is read).
 *   - The plan must already be on this device: one ponni_forward or
 *     ponni_plan_device_params call (which may allocate) puts it there, and
 *     a parameter change takes it off again; else PONNI_ERR_INVALID_ARGUMENT.
 *     That includes a change found in a host array shared with the plan
 *     (ponni_plan_share_layer_params with on_device = 0), reported with its
 *     own message.  A captured graph of this call keeps reading the device
 *     copy it was captured with: device-shared arrays are re-gathered by
 *     every replay, host-shared ones need a ponni_forward and a re-capture.
 *   - A batch whose GENERIC state buffers exceed the array gives
 *     PONNI_ERR_SHAPE (ponni_forward has no such limit).
 *   - All calls on one GPU share its array: calls that overlap in time on
 *     one GPU (different streams, or different plans without ordering) race.
 * Otherwise the arguments, results and asynchrony of ponni_forward. */
#define PONNI_NO_ALLOC_SCRATCH_BYTES (64ull << 20)
int ponni_forward_no_alloc(ponni_plan plan, const void* x, int64_t ld_in, void* y,
                           int64_t ld_out, int64_t batch, hipStream_t stream);

/* ponni_forward whose kernel dispatch stamps `start` and `stop` (events
 * created by the caller) with its own start and end, through the runtime's
 * extended launch, so that stop - start is the kernel's execution time with
 * no profiler attached.  A measurement aid with no counterpart in the
 * reference (it times forward_batch_parallel, ponni_Inference.h:352-389);
 * same arguments, errors and asynchrony as ponni_forward. */
int ponni_forward_timed(ponni_plan plan, const void* x, int64_t ld_in, void* y,
                        int64_t ld_out, int64_t batch, hipStream_t stream,
                        hipEvent_t start, hipEvent_t stop);

/* `steps` ponni_forward calls issued back to back from the library's host
 * code on `stream` (input and output pairs x[i % sets], y[i % sets]) between
 * two events; *ms_per_step = the elapsed time / steps.  A measurement aid
 * with no counterpart in the reference: the per-step time of the C ABI path
 * (host submission included) without an interpreter in between.
 * Synchronizes `stream`. */
int ponni_forward_steps(ponni_plan plan, const void* const* x, int64_t ld_in, void* const* y,
                        int64_t ld_out, int64_t batch, int32_t sets, int32_t steps,
                        hipStream_t stream, double* ms_per_step);

/* Source text of the kernel generated for a FUSED plan -- the counterpart of
 * the per-model executor the reference instantiates at compile time
 * (ponni_Inference.h:453-555) and of the emitted infer_batch body
 * (kokkos_nn/emitter.py:1537-1550).  Returns the length including the
 * terminating NUL (copying it when buf holds at least that many bytes), or
 * -1 for a non-FUSED plan. */
int64_t ponni_plan_kernel_source(ponni_plan plan, char* buf, int64_t len);

/* C++ text of an F32 / F64 plan's per-sample program: the op list of its
 * GENERIC lowering, which ponni_plan_device_model / ponni_plan_host_model
 * describe, as static constexpr members (dtype, num_ops, ops, steps,
 * tmp_features, saved_features, saved_total) for a struct that
 * ponni::forward_one_program (ponni_amd/include/ponni/device.h) runs with
 * each op expanded at compile time.  Generated model headers embed it for
 * infer_one, the reference emitter's per-model body with planned local
 * storage (kokkos_nn/emitter.py:1897-1901).  Returns the length including
 * the terminating NUL (copying it when buf holds at least that many bytes),
 * or -1 (other dtypes). */
int64_t ponni_plan_program_source(ponni_plan plan, char* buf, int64_t len);

/* Compile a FUSED plan's kernel with hipRTC now (no device needed; the result
 * is cached in-process and under $PONNI_JIT_CACHE or ~/.cache/ponni_hip) so the
 * first ponni_forward does not pay for it.  A no-op for the other paths.
 * Stands in for the compile step of building a reference model, which
 * happens when the application is compiled. */
int ponni_plan_compile(ponni_plan plan);

/* Launch configuration of the kernel generated for a FUSED or generated
 * NARROW plan (compiling it if needed; no device required): threads per
 * workgroup, batch columns per workgroup, and whether the grid is persistent
 * (at most the resident workgroups, each looping over tiles) or one
 * workgroup per tile.  With ponni_plan_kernel_source and
 * ponni_plan_device_params it lets a generated model header compile the
 * kernel ahead of time and launch it itself -- the counterpart of the
 * per-model kernel the reference's emitter writes into the header
 * (kokkos_nn/emitter.py:1537-1573). */
int ponni_plan_kernel_config(ponni_plan plan, int32_t* threads, int32_t* columns_per_block,
                             int32_t* persistent);

/* Device pointer to the plan's packed parameters in its kernel's layout
 * (uploading them first if they changed; synchronizes the device then):
 * the first argument of the generated kernel. */
int ponni_plan_device_params(ponni_plan plan, const void** params);

/* --- in-kernel (per-sample) inference ------------------------------------- */

/* Device-side description of a plan for application kernels that evaluate
 * one sample at a time (ponni_amd/include/ponni/device.h, ponni::forward_one):
 * the op list, epilogue steps and parameters of the plan's GENERIC lowering
 * (reference parameter layout), in device memory owned by the plan.  Stands
 * in for the reference's Inference::params (Params{saved_states, layers,
 * tmp1, tmp2}, ponni_Inference.h:127-149) as passed to
 * forward_batch_parallel_in_kernel (ponni_Inference.h:394-408, :592-604);
 * per-sample states live in the calling thread's private memory instead of
 * the [width, capacity] scratch. */
typedef struct ponni_device_model {
  const void* ops;    /* device op list (internal record, program.h) */
  const void* steps;  /* device epilogue steps */
  const void* params; /* device parameters, float (double for F64 plans) */
  int32_t num_ops;
  int32_t dtype;      /* ponni_dtype of the plan */
  int32_t num_inputs;
  int32_t num_outputs;
  int32_t max_width;  /* widest state of the chain */
  int32_t tmp_features[2];
  int32_t num_slots;   /* saved-state slots (get_num_saved_states()) */
  int32_t saved_total; /* features of all saved slots together */
  const int32_t* slot_rows; /* max(num_slots, 1) entries: slot s starts at
                               feature slot_rows[s] of the saved-state area */
} ponni_device_model;

/* Fill *out for `plan` (uploading its GENERIC form on first use and after
 * parameter changes; the pointers stay valid until the plan is destroyed).
 * Synchronizes the device when it uploads. */
int ponni_plan_device_model(ponni_plan plan, ponni_device_model* out);

/* Host execution-space models (create_inference_model(host execution space,
 * HostSpace, layers...), tests/unit/test_core_unit.cpp:380-404): the same
 * description with host pointers (the GENERIC op list and the parameters in
 * the compute type), for per-sample evaluation on the host with
 * ponni::forward_one.  Touches no device.  The pointers stay valid until the
 * plan's parameters change or the plan is destroyed.  F32 and F64 plans. */
int ponni_plan_host_model(ponni_plan plan, ponni_device_model* out);

/* forward_batch_parallel of a host execution-space model
 * (src/ponni_Inference.h:352-389 over a host execution space): x [num_inputs,
 * batch] and y [num_outputs, batch] in host memory with row strides ld_in and
 * ld_out, evaluated on the calling host by `threads` threads (0: one per
 * hardware thread) through the plan's GENERIC op list, synchronously.  F32
 * and F64 plans without external layers; the shape errors of ponni_forward. */
int ponni_forward_host(ponni_plan plan, const void* x, int64_t ld_in, void* y, int64_t ld_out, int64_t batch,
                       int32_t threads);

/* --- synthetic data (bench and tests) ------------------------------------- */

/* Fill n elements of a device buffer of `dtype` with the counter-based
 * synthetic stream: u64 = splitmix64(seed, tag, index); dist 0 = uniform on
 * [a, b) from the top 24 bits, dist 1 = normal(mean a, std b) by Box-Muller.
 * Asynchronous on `stream`. */
int ponni_fill_synthetic(void* x, int32_t dtype, int64_t n, uint64_t seed,
                         uint64_t tag, int32_t dist, double a, double b,
                         hipStream_t stream);

#define PONNI_DIST_UNIFORM 0
#define PONNI_DIST_NORMAL 1

/* Measured peaks of the current device, reported by bench.py beside the
 * published ones (no counterpart in the reference): the rates of a 1 GiB
 * device copy (bytes read + written per second), of a read-only pass over
 * the same 1 GiB, and of register-only loops
 * of v_mfma_f32_16x16x32_f16 and v_mfma_f32_16x16x4f32 with one 512-thread
 * workgroup per CU (the 16-bit FUSED kernels' occupancy); medians of a few
 * launches.  Also a copy of c1's traffic at c1's launch shape: 1,000,000
 * columns, 8 MB read from two rows and 4 MB written to one, 256-thread
 * workgroups with 16-byte accesses, 48 buffer sets in rotation, the mean of
 * the dispatches' own durations.  Allocates 2 GiB of device memory for the
 * call; synchronous. */
typedef struct ponni_peaks {
  double hbm_copy_gbps;
  double mfma_f16_tflops;
  double mfma_f32_tflops;
  double hbm_read_gbps;
  double hbm_copy_12mb_gbps; /* bytes read + written per second, c1-shaped copy */
  double copy_12mb_us;       /* its mean kernel duration */
} ponni_peaks;
int ponni_measure_peaks(ponni_peaks* out, hipStream_t stream);

/* --- .ponni weight files (host only) ------------------------------------- */

/* FNV-1a-64 of a byte string, utils/ponni_safetensors.h:25-32. */
uint64_t ponni_fnv1a64(const void* data, size_t size);

/* Fingerprint of the template weight schema of a layer chain, formatted
 * "fnv1a64:%016x"; Inference::weight_schema_fingerprint
 * (ponni_Inference.h:270-288).  `labels` are get_label() strings and
 * `trainable` the per-layer parameter counts exposed to training. */
int ponni_template_fingerprint(int32_t num_layers, const char* const* labels,
                               const int32_t* num_inputs,
                               const int32_t* num_outputs,
                               const int64_t* num_trainable, char* out,
                               size_t out_len);

/* Write a .ponni file holding one F32 (elem_size 4) or F64 (elem_size 8)
 * tensor named "parameters" of `count` elements; write_ponni_file
 * (utils/ponni_safetensors.h:350-407) as used by Inference::save_weights
 * (ponni_Inference.h:320-333). */
int ponni_file_write_parameters(const char* path, const char* model_fingerprint,
                                const void* values, int64_t count,
                                int32_t elem_size, const char* target);

/* Load and validate a .ponni file that must hold exactly one tensor
 * "parameters" of `count` elements of elem_size bytes bound to
 * `model_fingerprint`; PonniFile::load + PonniFile::validate
 * (utils/ponni_safetensors.h:187-347) as used by Inference::load_weights
 * (ponni_Inference.h:295-316).  Returns PONNI_ERR_IO with the reference's
 * rejection message in ponni_last_error() on failure. */
int ponni_file_read_parameters(const char* path, const char* model_fingerprint,
                               void* values, int64_t count, int32_t elem_size);

/* One named tensor of a multi-tensor .ponni file, as a generated model's
 * weight_specs() lists it (kokkos_nn/emitter.py:1438-1447): `offset` is the
 * tensor's first element in the model's flat parameter storage. */
typedef struct ponni_tensor_spec {
  const char* name;
  int32_t rank;
  int64_t shape[8];
  int64_t offset;
} ponni_tensor_spec;

/* Write tensors gathered from `storage` (double; stored as F32 when
 * stored_elem_size is 4, F64 when 8) into a .ponni file in name order with
 * the profile metadata; kokkos_nn/weights.py:95-153 and the generated
 * save_parameters (emitter.py:1754-1766). */
int ponni_file_write_tensors(const char* path, const char* model_fingerprint,
                             const ponni_tensor_spec* specs, int32_t num_specs,
                             const double* storage, int32_t stored_elem_size,
                             const char* source_framework, const char* target);

/* Load, validate against exactly these tensors and fingerprint, and scatter
 * every tensor into `storage` (double) at its offset; the generated
 * load_weights (emitter.py:1724-1752) over PonniFile::load / validate
 * (utils/ponni_safetensors.h:187-347). */
int ponni_file_read_tensors(const char* path, const char* model_fingerprint,
                            const ponni_tensor_spec* specs, int32_t num_specs,
                            double* storage, int32_t stored_elem_size);

#ifdef __cplusplus
}
#endif

#endif /* PONNI_HIP_H */
