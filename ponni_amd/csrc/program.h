// Internal "lane program": the plan compiler lowers a PONNI layer chain into a
// flat list of Op records that every kernel family interprets with uniform
// (scalar) control flow.  The record is shared by host and device code.
#pragma once

#ifdef __HIPCC_RTC__
using __hip_internal::int32_t;
using __hip_internal::int64_t;
using __hip_internal::uint64_t;
#else
#include <cstdint>
#endif

namespace ponni_hip {

// Pointwise step kinds.  A dense op carries the pointwise layers that follow
// it as an epilogue, exactly the fused block of ponni_Inference.h:412-444.
enum Act : int32_t {
  ACT_BIAS = 1,          // v + b[f]                         ponni_Bias.h:66-68
  ACT_RELU = 2,          // v > 0 ? v : 0                    ponni_Relu.h:49-51
  ACT_LEAKY_RELU = 3,    // v > 0 ? v : a*v                  ponni_LeakyRelu.h:53-55
  ACT_ELU = 4,           // v > 0 ? v : a*(exp(v)-1)         ponni_Elu.h:48-50
  ACT_SELU = 5,          //                                  ponni_Selu.h:45-49
  ACT_GELU_ERF = 6,      // 0.5 v (1 + erf(v/sqrt2))         ponni_Gelu.h:55-56
  ACT_GELU_TANH = 7,     // tanh form                        ponni_Gelu.h:48-53
  ACT_SILU = 8,          //                                  ponni_Silu.h:45-49
  ACT_SIGMOID = 9,       //                                  ponni_Sigmoid.h:45-49
  ACT_TANH = 10,         //                                  ponni_Tanh.h:44
  ACT_SOFTPLUS = 11,     // a = beta                         ponni_Softplus.h:44-50
  ACT_HARD_SIGMOID = 12, // a = alpha, b = beta              ponni_HardSigmoid.h:52-56
  ACT_HARD_SWISH = 13,   //                                  ponni_HardSwish.h:42-47
  ACT_MISH = 14,         //                                  ponni_Mish.h:44-52
  // Unary operations of generated graphs (kokkos_nn/emitter.py:218-258).
  ACT_ABS = 20,
  ACT_NEG = 21,
  ACT_EXP = 22,
  ACT_LOG = 23,
  ACT_SQRT = 24,
  ACT_RECIPROCAL = 25,
  ACT_SOFTSIGN = 26,          // v / (1 + |v|)
  ACT_CELU = 27,              // v > 0 ? v : a*(exp(v/a)-1)
  ACT_THRESHOLDED_RELU = 28,  // v > a ? v : 0
  ACT_ERF = 29,
  ACT_SELU_AG = 30,           // b * (v > 0 ? v : a*(exp(v)-1)), generated Selu(alpha, gamma)
  // ACT_ABS + ponni_unary_op for the rest (interpreter.py:15-117):
  ACT_ACOS = 31,
  ACT_ACOSH = 32,
  ACT_ASIN = 33,
  ACT_ASINH = 34,
  ACT_ATAN = 35,
  ACT_ATANH = 36,
  ACT_CEIL = 37,
  ACT_COS = 38,
  ACT_COSH = 39,
  ACT_FLOOR = 40,
  ACT_SIN = 41,
  ACT_SINH = 42,
  ACT_TAN = 43,
  ACT_ROUND = 44,       // nearest, ties to even
  ACT_SIGN = 45,        // -1 / 0 / 1, NaN kept
  ACT_IS_NAN = 46,      // 1 / 0
  ACT_IS_INF = 47,      // 1 / 0; a = detect_negative, b = detect_positive
  ACT_NOT = 48,         // v == 0 ? 1 : 0
  ACT_NONZERO = 49,     // v != 0 ? 1 : 0 (Cast to bool)
  // Element-wise op with a constant vector c = params[off + f] (generated
  // Add/Sub/Mul/Div/Min/Max/Pow with one constant operand, emitter.py:261-275).
  // ACT_BIAS doubles as v + c.
  ACT_SUB_C = 60,   // v - c
  ACT_RSUB_C = 61,  // c - v
  ACT_MUL_C = 62,   // v * c
  ACT_DIV_C = 63,   // v / c
  ACT_RDIV_C = 64,  // c / v
  ACT_MIN_C = 65,   // v < c ? v : c
  ACT_RMIN_C = 66,  // c < v ? c : v
  ACT_MAX_C = 67,   // v > c ? v : c
  ACT_RMAX_C = 68,  // c > v ? c : v
  ACT_POW_C = 69,   // pow(v, c)
  ACT_RPOW_C = 70,  // pow(c, v)
  ACT_CBIN = 71     // ponni_binary_op a (comparisons, logic, PRelu) of v and c; b != 0: c on the left
};

// Steps that read a per-feature parameter vector at Step::off.
constexpr bool act_has_param(int act) { return act == ACT_BIAS || (act >= ACT_SUB_C && act <= ACT_CBIN); }

struct Step {
  int32_t act;   // Act
  int32_t off;   // parameter offset of the bias vector (ACT_BIAS only)
  double a;      // scalar attribute (slope, alpha, beta), exact for F64 plans
  double b;      // second scalar attribute
};

enum OpCode : int32_t {
  OP_DENSE = 1,       // out = epilogue(W^T in)                     Matvec + pointwise
  OP_POINTWISE = 2,   // state = epilogue(state), in place          lone pointwise layer
  OP_LAYER_NORM = 3,  // two-pass mean/var, gamma/beta              ponni_LayerNorm.h:76-99
  OP_SOFTMAX = 4,     //                                            ponni_Softmax.h:45-56
  OP_LOG_SOFTMAX = 5, //                                            ponni_LogSoftmax.h:45-57
  OP_MIN_MAX = 6,     //                                            ponni_MinMaxNorm.h:67-84
  OP_SAVE = 7,        // saved[slot] = state                        ponni_Save_State.h:57-67
  OP_ADD = 8,         // state = state + saved[slot]                ponni_Binop_Add.h:57-68
  OP_CONCAT = 9,      // state = [state; saved] or [saved; state]   ponni_Binop_Concatenate.h:63-86
  OP_PROJ_ADD = 10,   // state = state + (b + W^T saved[slot])      ponni_Binop_Projection_Add.h:81-95
  // Generated-graph operations (kokkos_nn/emitter.py).
  OP_LOAD = 11,       // state = saved[slot]
  OP_BINARY = 12,     // state = op(state, saved) / op(saved, state); aux = BinaryAux bits
  OP_REDUCE = 13,     // state[0] = reduce(state[0..n_in)); aux = ponni_reduce_op   emitter.py:475-547
  // A caller-implemented layer (PONNI_LAYER_EXTERNAL): aux = the caller's
  // index, boff = PONNI_FLAG_EXT_* bits | EXT_ALSO_TMP1.
  OP_EXTERNAL = 14,
  // state = cond != 0 ? a : b (interpreter.py:178-183 Where / CompareSelect); aux =
  // SelectAux bits; slot = the first saved operand's slot, f0 = the second's;
  // woff / boff = parameter offsets of the first / second constant operand.
  OP_SELECT = 15
};

// OP_SELECT's aux: operand sources (2 bits each: 0 state, 1 first slot
// operand, 2 second slot operand, 3 constant) of cond, a, b, then the
// one-feature (broadcast) flags.
enum SelectAux : int32_t {
  SEL_SRC_BITS = 2,
  SEL_COND_SCALAR = 1 << 6,
  SEL_A_SCALAR = 1 << 7,
  SEL_B_SCALAR = 1 << 8
};
constexpr int sel_src(int aux, int operand) { return (aux >> (2 * operand)) & 3; }

// OP_EXTERNAL's boff: a leading saving layer also fills tmp1
// (ponni_Inference.h:499-514).
constexpr int32_t EXT_ALSO_TMP1 = 1 << 8;

// OP_BINARY's aux: bits 0-7 ponni_binary_op, then these flags.
enum BinaryAux : int32_t {
  BIN_SAVED_LEFT = 1 << 8,    // saved operand is the left one
  BIN_SAVED_SCALAR = 1 << 9,  // saved operand has one feature (broadcast)
  BIN_STATE_SCALAR = 1 << 10  // state operand has one feature (broadcast)
};

// OP_DENSE's aux: the first epilogue step is a bias that seeds the sum
// (generated Dense: sum = bias; sum += W x, emitter.py:701-710).
constexpr int32_t DENSE_BIAS_FIRST = 1;

// Buffers of the generic (HBM scratch) path, chosen at plan time exactly as
// traverse_mixed_batch_parallel picks them (ponni_Inference.h:453-555).
enum Buffer : int32_t {
  BUF_INPUT = 0,
  BUF_OUTPUT = 1,
  BUF_TMP1 = 2,
  BUF_TMP2 = 3,
  BUF_SAVED = 4  // BUF_SAVED + slot
};

struct Op {
  int32_t code;       // OpCode
  int32_t n_in;       // features read from the main state
  int32_t n_out;      // features written to the main state
  int32_t slot;       // saved-state slot (SAVE/ADD/CONCAT/PROJ_ADD)
  int32_t aux;        // CONCAT: 1 = after; PROJ_ADD: NSAVE; BINARY: BinaryAux; REDUCE: op;
                      // DENSE: DENSE_BIAS_FIRST
  int32_t woff;       // offset of W / gamma in the path's parameter buffer
  int32_t boff;       // offset of bias / beta
  int32_t epi_begin;  // first Step of the epilogue
  int32_t epi_count;  // number of Steps
  int32_t src;        // generic path: input buffer
  int32_t dst;        // generic path: output buffer
  double f0, f1, f2;  // scalar attributes (epsilon, out_min, out_max), exact for F64 plans
};

// Saved-state slot indices a plan may use: 0 .. kMaxSlots - 1.  Slots are
// sized from the plan (one area, Bufs in generic_ops.h); the bound only
// keeps the per-slot table small for a stray index.
constexpr int kMaxSlots = 4096;

}  // namespace ponni_hip
