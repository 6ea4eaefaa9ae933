// Host side of libponni_hip: layer-chain validation, lowering to the lane
// program, scratch planning, parameter packing and the C ABI entry points.
//
// Reference behaviour restated here:
//   - validation         src/ponni_Inference.h:719-737 plus each layer's validate()
//   - block planning     src/ponni_Inference.h:56-85 (dense + following pointwise)
//   - buffer selection   src/ponni_Inference.h:453-555 (tmp1/tmp2/saved ping-pong)
//   - scratch sizing     src/ponni_Inference.h:92-122, :204-223
//   - forward contract   src/ponni_Inference.h:352-389
#include "plan.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <sstream>
#include <string>

#include "fused.h"
#include "host_half.h"

using namespace ponni_hip;

namespace {

thread_local std::string g_last_error;

int fail(int status, std::string const& message) {
  g_last_error = message;
  return status;
}

bool is_pointwise(int kind) {
  return kind == PONNI_LAYER_BIAS || (kind >= PONNI_LAYER_RELU && kind <= PONNI_LAYER_MISH) ||
         kind == PONNI_LAYER_UNARY || kind == PONNI_LAYER_CONST_BINARY;
}

bool is_dense(int kind) { return kind == PONNI_LAYER_MATVEC || kind == PONNI_LAYER_DENSE; }

// Kinds that read a saved slot.
bool reads_slot(int kind) {
  return kind == PONNI_LAYER_BINOP_ADD || kind == PONNI_LAYER_BINOP_CONCATENATE ||
         kind == PONNI_LAYER_BINOP_PROJECTION_ADD || kind == PONNI_LAYER_LOAD_STATE || kind == PONNI_LAYER_BINARY ||
         kind == PONNI_LAYER_SELECT;
}

bool is_graph_kind(int kind) { return kind >= PONNI_LAYER_DENSE && kind <= PONNI_LAYER_SELECT; }

// The operands of a PONNI_LAYER_SELECT (cond, a, b): where each comes from
// (PONNI_SELECT_*), its slot when saved (the first saved operand is
// d.slot, the second attr[1]), whether it is one feature, and the number
// of constant operands.
struct SelectOperands {
  int src[3];
  int slot[3];
  bool scalar[3];
  int num_slots = 0;
  int num_const = 0;
};
SelectOperands select_operands(ponni_layer_desc const& d) {
  SelectOperands o{};
  int const scalar_bits[3] = {PONNI_SELECT_COND_SCALAR, PONNI_SELECT_A_SCALAR, PONNI_SELECT_B_SCALAR};
  for (int k = 0; k < 3; k++) {
    o.src[k] = (d.flags >> (2 * k)) & 3;
    o.slot[k] = -1;
    o.scalar[k] = (d.flags & scalar_bits[k]) != 0;
    if (o.src[k] == PONNI_SELECT_SLOT) o.slot[k] = o.num_slots++ == 0 ? d.slot : static_cast<int>(d.attr[1]);
    if (o.src[k] == PONNI_SELECT_CONST) o.num_const++;
  }
  return o;
}

bool is_save(int kind) { return kind == PONNI_LAYER_SAVE_STATE; }

bool is_binop(int kind) {
  return kind == PONNI_LAYER_BINOP_ADD || kind == PONNI_LAYER_BINOP_CONCATENATE ||
         kind == PONNI_LAYER_BINOP_PROJECTION_ADD;
}

bool known_kind(int kind) {
  return kind == PONNI_LAYER_MATVEC || is_pointwise(kind) ||
         (kind >= PONNI_LAYER_SOFTMAX && kind <= PONNI_LAYER_MIN_MAX_NORM) || is_save(kind) ||
         is_binop(kind) || is_graph_kind(kind) || kind == PONNI_LAYER_EXTERNAL;
}

bool ext_saves(ponni_layer_desc const& d) {
  return d.kind == PONNI_LAYER_EXTERNAL && (d.flags & PONNI_FLAG_EXT_SAVE);
}
bool ext_reads(ponni_layer_desc const& d) {
  return d.kind == PONNI_LAYER_EXTERNAL && (d.flags & PONNI_FLAG_EXT_BINOP);
}

char const* label_of(int kind) {
  switch (kind) {
    case PONNI_LAYER_EXTERNAL: return "External";
    case PONNI_LAYER_MATVEC: return "Matvec";
    case PONNI_LAYER_BIAS: return "Bias";
    case PONNI_LAYER_RELU: return "ReLU";
    case PONNI_LAYER_LEAKY_RELU: return "LeakyReLU";
    case PONNI_LAYER_ELU: return "ELU";
    case PONNI_LAYER_SELU: return "SELU";
    case PONNI_LAYER_GELU: return "GELU";
    case PONNI_LAYER_SILU: return "SiLU";
    case PONNI_LAYER_SIGMOID: return "Sigmoid";
    case PONNI_LAYER_TANH: return "Tanh";
    case PONNI_LAYER_SOFTPLUS: return "Softplus";
    case PONNI_LAYER_HARD_SIGMOID: return "HardSigmoid";
    case PONNI_LAYER_HARD_SWISH: return "HardSwish";
    case PONNI_LAYER_MISH: return "Mish";
    case PONNI_LAYER_SOFTMAX: return "Softmax";
    case PONNI_LAYER_LOG_SOFTMAX: return "LogSoftmax";
    case PONNI_LAYER_LAYER_NORM: return "LayerNorm";
    case PONNI_LAYER_MIN_MAX_NORM: return "MinMaxNorm";
    case PONNI_LAYER_SAVE_STATE: return "Save_State";
    case PONNI_LAYER_BINOP_ADD: return "Binop_Add";
    case PONNI_LAYER_BINOP_CONCATENATE: return "Binop_Concatenate";
    case PONNI_LAYER_BINOP_PROJECTION_ADD: return "Binop_Projection_Add";
    case PONNI_LAYER_DENSE: return "Dense";
    case PONNI_LAYER_LOAD_STATE: return "Load_State";
    case PONNI_LAYER_BINARY: return "Binary";
    case PONNI_LAYER_REDUCE: return "Reduce";
    case PONNI_LAYER_UNARY: return "Unary";
    case PONNI_LAYER_CONST_BINARY: return "Const_Binary";
    case PONNI_LAYER_SELECT: return "Select";
    default: return "?";
  }
}

int64_t param_count(ponni_layer_desc const& d) {
  switch (d.kind) {
    case PONNI_LAYER_MATVEC: return int64_t(d.n_in) * d.n_out;
    case PONNI_LAYER_BIAS: return d.n_in;
    case PONNI_LAYER_LAYER_NORM: return 2 * int64_t(d.n_in);
    case PONNI_LAYER_BINOP_PROJECTION_ADD: return int64_t(d.n_aux) * d.n_in + d.n_in;
    case PONNI_LAYER_DENSE: return int64_t(d.n_out) * d.n_in + ((d.flags & PONNI_FLAG_DENSE_BIAS) ? d.n_out : 0);
    case PONNI_LAYER_CONST_BINARY: return d.n_in;
    case PONNI_LAYER_SELECT: return int64_t(select_operands(d).num_const) * d.n_out;
    default: return 0;
  }
}

// Each layer's own validate() plus the chain check of Inference::validate.
int validate_chain(ponni_layer_desc const* layers, int n) {
  std::string where;
  std::vector<int> saved_size(kMaxSlots, 0);
  std::vector<char> saved_seen(kMaxSlots, 0);
  for (int i = 0; i < n; i++) {
    ponni_layer_desc const& d = layers[i];
    where = "layer " + std::to_string(i) + " (" + label_of(d.kind) + "): ";
    if (!known_kind(d.kind)) return fail(PONNI_ERR_INVALID_ARGUMENT, where + "unknown layer kind " + std::to_string(d.kind));
    if (d.n_in <= 0 || d.n_out <= 0) return fail(PONNI_ERR_INVALID_MODEL, where + "num_inputs and num_outputs must be > 0");
    bool const same_width = !is_dense(d.kind) && d.kind != PONNI_LAYER_BINOP_CONCATENATE &&
                            d.kind != PONNI_LAYER_LOAD_STATE && d.kind != PONNI_LAYER_BINARY &&
                            d.kind != PONNI_LAYER_REDUCE && d.kind != PONNI_LAYER_EXTERNAL &&
                            d.kind != PONNI_LAYER_SELECT;
    if (same_width && d.n_in != d.n_out) return fail(PONNI_ERR_INVALID_MODEL, where + "input/output size mismatch");
    if (is_save(d.kind) || reads_slot(d.kind) || ext_saves(d) || ext_reads(d)) {
      if (d.slot < 0 || d.slot >= kMaxSlots) return fail(PONNI_ERR_INVALID_MODEL, where + "saved-state index out of range [0," + std::to_string(kMaxSlots) + ")");
    }
    if (ext_saves(d)) {
      saved_size[d.slot] = d.n_out;
      saved_seen[d.slot] = true;
    }
    if (ext_reads(d) && !saved_seen[d.slot])
      return fail(PONNI_ERR_INVALID_MODEL, where + "reads saved state " + std::to_string(d.slot) + " before any save wrote it");
    if (d.kind == PONNI_LAYER_EXTERNAL && (ext_saves(d) && ext_reads(d)))
      return fail(PONNI_ERR_INVALID_MODEL, where + "a layer cannot both save and read a saved state");
    switch (d.kind) {
      case PONNI_LAYER_ELU:
        if (!(d.attr[0] > 0)) return fail(PONNI_ERR_INVALID_MODEL, where + "ELU alpha must be > 0");
        break;
      case PONNI_LAYER_SOFTPLUS:
        if (!(d.attr[0] > 0)) return fail(PONNI_ERR_INVALID_MODEL, where + "Softplus beta must be > 0");
        break;
      case PONNI_LAYER_HARD_SIGMOID:
        if (!(d.attr[0] > 0)) return fail(PONNI_ERR_INVALID_MODEL, where + "HardSigmoid alpha must be > 0");
        break;
      case PONNI_LAYER_LAYER_NORM:
        if (!(d.attr[0] > 0)) return fail(PONNI_ERR_INVALID_MODEL, where + "LayerNorm epsilon must be > 0");
        break;
      case PONNI_LAYER_MIN_MAX_NORM:
        if (!(d.attr[1] > d.attr[0])) return fail(PONNI_ERR_INVALID_MODEL, where + "MinMaxNorm requires out_max > out_min");
        if (!(d.attr[2] > 0)) return fail(PONNI_ERR_INVALID_MODEL, where + "MinMaxNorm epsilon must be > 0");
        break;
      case PONNI_LAYER_SAVE_STATE:
        saved_size[d.slot] = d.n_in;
        saved_seen[d.slot] = true;
        break;
      case PONNI_LAYER_LOAD_STATE:
      case PONNI_LAYER_BINARY: {
        if (!saved_seen[d.slot])
          return fail(PONNI_ERR_INVALID_MODEL, where + "reads saved state " + std::to_string(d.slot) + " before any Save_State wrote it");
        int const saved = saved_size[d.slot];
        if (d.kind == PONNI_LAYER_LOAD_STATE && d.n_out != saved)
          return fail(PONNI_ERR_INVALID_MODEL, where + "num outputs != the saved state's width");
        if (d.kind == PONNI_LAYER_BINARY) {
          int const op = static_cast<int>(d.attr[0]);
          if (d.attr[0] != op || op < PONNI_BINARY_ADD || op > PONNI_BINARY_PRELU)
            return fail(PONNI_ERR_INVALID_MODEL, where + "unknown binary operation");
          if (d.n_aux != saved) return fail(PONNI_ERR_INVALID_MODEL, where + "n_aux != the saved state's width");
          if ((saved != 1 && saved != d.n_out) || (d.n_in != 1 && d.n_in != d.n_out) ||
              (d.n_out != std::max(d.n_in, saved)))
            return fail(PONNI_ERR_INVALID_MODEL, where + "unsupported broadcasting: operand sizes " + std::to_string(d.n_in) +
                                                     " and " + std::to_string(saved) + ", output size " +
                                                     std::to_string(d.n_out));
        }
        break;
      }
      case PONNI_LAYER_SELECT: {
        SelectOperands const o = select_operands(d);
        int states = 0;
        for (int k = 0; k < 3; k++) {
          if (o.src[k] > PONNI_SELECT_CONST) return fail(PONNI_ERR_INVALID_MODEL, where + "unknown operand source");
          states += o.src[k] == PONNI_SELECT_STATE;
        }
        if (states != 1) return fail(PONNI_ERR_INVALID_MODEL, where + "exactly one operand is the state");
        if (o.src[0] == PONNI_SELECT_CONST) return fail(PONNI_ERR_INVALID_MODEL, where + "the condition is not a constant");
        if (o.num_slots == 2 && (d.attr[1] != static_cast<int>(d.attr[1]) || d.attr[1] < 0 || d.attr[1] >= kMaxSlots))
          return fail(PONNI_ERR_INVALID_MODEL, where + "saved-state index out of range [0," + std::to_string(kMaxSlots) + ")");
        for (int k = 0; k < 3; k++) {
          int width = d.n_out;
          if (o.src[k] == PONNI_SELECT_STATE) width = d.n_in;
          if (o.src[k] == PONNI_SELECT_SLOT) {
            if (!saved_seen[o.slot[k]])
              return fail(PONNI_ERR_INVALID_MODEL, where + "reads saved state " + std::to_string(o.slot[k]) +
                                                       " before any Save_State wrote it");
            width = saved_size[o.slot[k]];
          }
          if (o.src[k] == PONNI_SELECT_CONST && o.scalar[k])
            return fail(PONNI_ERR_INVALID_MODEL, where + "a constant operand holds n_out values");
          if ((width != 1 && width != d.n_out) || o.scalar[k] != (width == 1 && d.n_out > 1))
            return fail(PONNI_ERR_INVALID_MODEL, where + "unsupported broadcasting: an operand of " +
                                                     std::to_string(width) + " features, output size " +
                                                     std::to_string(d.n_out));
        }
        break;
      }
      case PONNI_LAYER_REDUCE: {
        int const op = static_cast<int>(d.attr[0]);
        if (d.attr[0] != op || op < PONNI_REDUCE_SUM || op > PONNI_REDUCE_PROD)
          return fail(PONNI_ERR_INVALID_MODEL, where + "unknown reduction");
        if (d.n_out != 1) return fail(PONNI_ERR_INVALID_MODEL, where + "a reduction has one output");
        break;
      }
      case PONNI_LAYER_UNARY: {
        int const op = static_cast<int>(d.attr[0]);
        if (d.attr[0] != op || op < PONNI_UNARY_ABS || op > PONNI_UNARY_NONZERO)
          return fail(PONNI_ERR_INVALID_MODEL, where + "unknown unary operation");
        if (op == PONNI_UNARY_CELU && !(d.attr[1] != 0)) return fail(PONNI_ERR_INVALID_MODEL, where + "Celu alpha must be nonzero");
        break;
      }
      case PONNI_LAYER_CONST_BINARY: {
        int const op = static_cast<int>(d.attr[0]);
        if (d.attr[0] != op || op < PONNI_BINARY_ADD || op > PONNI_BINARY_PRELU)
          return fail(PONNI_ERR_INVALID_MODEL, where + "unknown binary operation");
        break;
      }
      case PONNI_LAYER_BINOP_ADD:
      case PONNI_LAYER_BINOP_CONCATENATE:
      case PONNI_LAYER_BINOP_PROJECTION_ADD: {
        if (i == 0) return fail(PONNI_ERR_INVALID_MODEL, where + "a binary layer cannot be first: no state has been saved");
        if (!saved_seen[d.slot]) return fail(PONNI_ERR_INVALID_MODEL, where + "reads saved state " + std::to_string(d.slot) + " before any Save_State wrote it");
        int const saved = saved_size[d.slot];
        if (d.kind == PONNI_LAYER_BINOP_ADD && saved != d.n_in)
          return fail(PONNI_ERR_INVALID_MODEL, where + "Saved layer num inputs != this layer's num inputs");
        if (d.kind == PONNI_LAYER_BINOP_CONCATENATE && d.n_out != saved + d.n_in)
          return fail(PONNI_ERR_INVALID_MODEL, where + "this layer's num outputs != this layer's num inputs + saved layer's num inputs");
        if (d.kind == PONNI_LAYER_BINOP_PROJECTION_ADD && (d.n_aux <= 0 || d.n_aux != saved))
          return fail(PONNI_ERR_INVALID_MODEL, where + "saved layer size incompatible with projection weights");
        break;
      }
      default:
        break;
    }
    if (i + 1 < n && d.n_out != layers[i + 1].n_in)
      return fail(PONNI_ERR_INVALID_MODEL, where + "This layer's num outputs != next layer's num inputs");
  }
  return PONNI_OK;
}

Step make_step(ponni_layer_desc const& d) {
  Step s{};
  switch (d.kind) {
    case PONNI_LAYER_BIAS: s.act = ACT_BIAS; break;
    case PONNI_LAYER_RELU: s.act = ACT_RELU; break;
    case PONNI_LAYER_LEAKY_RELU: s.act = ACT_LEAKY_RELU; s.a = d.attr[0]; break;
    case PONNI_LAYER_ELU: s.act = ACT_ELU; s.a = d.attr[0]; break;
    case PONNI_LAYER_SELU: s.act = ACT_SELU; break;
    case PONNI_LAYER_GELU: s.act = (d.flags & PONNI_FLAG_GELU_APPROXIMATE) ? ACT_GELU_TANH : ACT_GELU_ERF; break;
    case PONNI_LAYER_SILU: s.act = ACT_SILU; break;
    case PONNI_LAYER_SIGMOID: s.act = ACT_SIGMOID; break;
    case PONNI_LAYER_TANH: s.act = ACT_TANH; break;
    case PONNI_LAYER_SOFTPLUS: s.act = ACT_SOFTPLUS; s.a = d.attr[0]; break;
    case PONNI_LAYER_HARD_SIGMOID: s.act = ACT_HARD_SIGMOID; s.a = d.attr[0]; s.b = d.attr[1]; break;
    case PONNI_LAYER_HARD_SWISH: s.act = ACT_HARD_SWISH; break;
    case PONNI_LAYER_MISH: s.act = ACT_MISH; break;
    case PONNI_LAYER_UNARY:
      s.act = ACT_ABS + static_cast<int>(d.attr[0]);  // ponni_unary_op order
      s.a = d.attr[1];
      s.b = d.attr[2];
      break;
    case PONNI_LAYER_CONST_BINARY: {
      bool const left = d.flags & PONNI_FLAG_CONST_LEFT;
      switch (static_cast<int>(d.attr[0])) {
        case PONNI_BINARY_ADD: s.act = ACT_BIAS; break;
        case PONNI_BINARY_SUB: s.act = left ? ACT_RSUB_C : ACT_SUB_C; break;
        case PONNI_BINARY_MUL: s.act = ACT_MUL_C; break;
        case PONNI_BINARY_DIV: s.act = left ? ACT_RDIV_C : ACT_DIV_C; break;
        case PONNI_BINARY_MIN: s.act = left ? ACT_RMIN_C : ACT_MIN_C; break;
        case PONNI_BINARY_MAX: s.act = left ? ACT_RMAX_C : ACT_MAX_C; break;
        case PONNI_BINARY_POW: s.act = left ? ACT_RPOW_C : ACT_POW_C; break;
        default:
          s.act = ACT_CBIN;
          s.a = d.attr[0];
          s.b = left ? 1 : 0;
          break;
      }
      break;
    }
    default: break;
  }
  return s;
}

int round_up(int v, int m) { return (v + m - 1) / m * m; }

// GENERIC and LAYERED plans share the op list, the reference parameter
// layout and the HBM scratch.
bool generic_layout(ponni_plan_s const& p) { return p.path == PONNI_PATH_GENERIC || p.path == PONNI_PATH_LAYERED; }

// Rows of the saved-slot area (generic_ops.h Bufs): slot s after slots
// 0 .. s-1, each get_saved_state_size<s>() rows high.
void set_slot_rows(ponni_plan_s& p) {
  p.saved_features.resize(p.num_slots, 0);
  p.slot_rows.assign(std::max(p.num_slots, 1), 0);
  int32_t row = 0;
  for (int s = 0; s < p.num_slots; s++) {
    p.slot_rows[s] = row;
    row += p.saved_features[s];
  }
  p.saved_total = row;
}

std::vector<int32_t> contractions_over_input(ponni_plan_s const& p) {
  bool const half = p.dtype == PONNI_F16 || p.dtype == PONNI_BF16;
  if (p.path != PONNI_PATH_FUSED || half || p.layers.empty() || p.layers.front().n_in % 16 == 0) return {};
  bool cur = true;                 // the state holds the input
  std::vector<char> saved(std::max(p.num_slots, 1), 0);  // slot s holds the input
  std::vector<int32_t> woffs;
  for (Op const& op : p.ops) {
    switch (op.code) {
      case OP_DENSE:
        if (cur) woffs.push_back(op.woff);
        cur = false;
        break;
      case OP_SAVE: saved[op.slot] = cur; break;
      case OP_LOAD: cur = saved[op.slot]; break;
      case OP_PROJ_ADD:
        if (cur) return {};
        if (saved[op.slot]) woffs.push_back(op.woff);
        break;
      case OP_ADD:
      case OP_CONCAT:
      case OP_BINARY:
      case OP_SELECT:
      case OP_EXTERNAL:
        if (cur || saved[op.slot] || (op.code == OP_SELECT && op.f0 >= 0 && saved[static_cast<int>(op.f0)]))
          return {};
        break;
      default:
        if (cur) return {};
        break;
    }
  }
  if (cur) return {};
  return woffs;
}

// Per-path packed size and layout of one layer's parameters.
// GENERIC: reference layout.  NARROW: padded to the width class W.
// MFMA: dense weights in A-fragment order, vectors padded to 16.
int64_t packed_size(ponni_plan_s const& p, ponni_layer_desc const& d) {
  int const W = p.width_class;
  switch (p.path) {
    case PONNI_PATH_NARROW:
      switch (d.kind) {
        case PONNI_LAYER_MATVEC: return int64_t(W) * W;
        case PONNI_LAYER_DENSE: return int64_t(W) * W + ((d.flags & PONNI_FLAG_DENSE_BIAS) ? W : 0);
        case PONNI_LAYER_CONST_BINARY: return W;
        case PONNI_LAYER_BIAS: return W;
        case PONNI_LAYER_LAYER_NORM: return 2 * W;
        case PONNI_LAYER_BINOP_PROJECTION_ADD: return int64_t(W) * W + W;
        case PONNI_LAYER_SELECT: return int64_t(select_operands(d).num_const) * W;
        default: return 0;
      }
    case PONNI_PATH_MFMA:
    case PONNI_PATH_FUSED: {
      auto tiles = [](int n) { return (n + 15) / 16; };
      if (p.path == PONNI_PATH_FUSED && (p.dtype == PONNI_F16 || p.dtype == PONNI_BF16)) {
        // Dense blocks: one 1 KB fragment (256 four-byte units) per output tile
        // and 32-feature step; vectors stay fp32.
        auto steps = [&](int n) { return (tiles(n) + 1) / 2; };
        switch (d.kind) {
          case PONNI_LAYER_MATVEC: return int64_t(steps(d.n_in)) * tiles(d.n_out) * 256;
          case PONNI_LAYER_DENSE:
            return int64_t(steps(d.n_in)) * tiles(d.n_out) * 256 +
                   ((d.flags & PONNI_FLAG_DENSE_BIAS) ? round_up(d.n_out, 16) : 0);
          case PONNI_LAYER_CONST_BINARY:
          case PONNI_LAYER_BIAS: return round_up(d.n_in, 16);
          case PONNI_LAYER_LAYER_NORM: return 2 * round_up(d.n_in, 16);
          case PONNI_LAYER_BINOP_PROJECTION_ADD:
            return int64_t(steps(d.n_aux)) * tiles(d.n_in) * 256 + round_up(d.n_in, 16);
          case PONNI_LAYER_SELECT: return int64_t(select_operands(d).num_const) * round_up(d.n_out, 16);
          default: return 0;
        }
      }
      switch (d.kind) {
        case PONNI_LAYER_MATVEC: return int64_t(tiles(d.n_in)) * tiles(d.n_out) * 256;
        case PONNI_LAYER_DENSE:
          return int64_t(tiles(d.n_in)) * tiles(d.n_out) * 256 +
                 ((d.flags & PONNI_FLAG_DENSE_BIAS) ? round_up(d.n_out, 16) : 0);
        case PONNI_LAYER_CONST_BINARY:
        case PONNI_LAYER_BIAS: return round_up(d.n_in, 16);
        case PONNI_LAYER_LAYER_NORM: return 2 * round_up(d.n_in, 16);
        case PONNI_LAYER_BINOP_PROJECTION_ADD:
          return int64_t(tiles(d.n_aux)) * tiles(d.n_in) * 256 + round_up(d.n_in, 16);
        case PONNI_LAYER_SELECT: return int64_t(select_operands(d).num_const) * round_up(d.n_out, 16);
        default: return 0;
      }
    }
    default:
      return param_count(d);
  }
}

// Packed length of a per-feature vector of n features in the path's layout.
int64_t vec_size(ponni_plan_s const& p, int n) {
  switch (p.path) {
    case PONNI_PATH_GENERIC:
    case PONNI_PATH_LAYERED: return n;
    case PONNI_PATH_NARROW: return p.width_class;
    default: return round_up(n, 16);
  }
}

// Lower the chain into ops; mirrors the traversal of ponni_Inference.h:453-555.
void lower(ponni_plan_s& p) {
  int const L = static_cast<int>(p.layers.size());
  p.ops.clear();
  p.steps.clear();
  p.layer_param_offset.assign(L, 0);
  int64_t off = 0;
  for (int i = 0; i < L; i++) {
    p.layer_param_offset[i] = off;
    off += packed_size(p, p.layers[i]);
  }
  p.packed_elements = off;

  int vec_stride_ln = 0;  // offset of beta after gamma
  bool in_tmp1 = false;
  int tmp_max[2] = {0, 0};
  p.num_fused_blocks = 0;
  for (int i = 0; i < L;) {
    ponni_layer_desc const& d = p.layers[i];
    Op op{};
    op.n_in = d.n_in;
    op.n_out = d.n_out;
    op.slot = d.slot;
    op.woff = static_cast<int32_t>(p.layer_param_offset[i]);
    if (is_dense(d.kind)) {
      int end = i + 1;
      while (end < L && is_pointwise(p.layers[end].kind)) end++;
      op.code = OP_DENSE;
      op.epi_begin = static_cast<int32_t>(p.steps.size());
      op.epi_count = end - (i + 1);
      if (d.kind == PONNI_LAYER_DENSE && (d.flags & PONNI_FLAG_DENSE_BIAS)) {
        // Generated Dense: its bias (stored after W) seeds the sum.
        Step s{};
        s.act = ACT_BIAS;
        s.off = static_cast<int32_t>(p.layer_param_offset[i] + packed_size(p, d) - vec_size(p, d.n_out));
        p.steps.push_back(s);
        op.epi_count++;
        op.aux = DENSE_BIAS_FIRST;
      }
      for (int j = i + 1; j < end; j++) {
        Step s = make_step(p.layers[j]);
        s.off = static_cast<int32_t>(p.layer_param_offset[j]);
        p.steps.push_back(s);
      }
      op.n_out = p.layers[end - 1].n_out;
      p.num_fused_blocks++;
      if (i == 0) {
        op.src = BUF_INPUT;
        if (end == L) {
          op.dst = BUF_OUTPUT;
        } else {
          op.dst = BUF_TMP1;
          tmp_max[0] = std::max(tmp_max[0], d.n_out);
          in_tmp1 = true;
        }
      } else {
        op.src = in_tmp1 ? BUF_TMP1 : BUF_TMP2;
        if (end == L) {
          op.dst = BUF_OUTPUT;
        } else {
          bool const out_tmp1 = !in_tmp1;
          op.dst = out_tmp1 ? BUF_TMP1 : BUF_TMP2;
          tmp_max[out_tmp1 ? 0 : 1] = std::max(tmp_max[out_tmp1 ? 0 : 1], d.n_out);
          in_tmp1 = out_tmp1;
        }
      }
      p.ops.push_back(op);
      i = end;
      continue;
    }
    // Barrier (or lone pointwise) layer.
    switch (d.kind) {
      case PONNI_LAYER_LAYER_NORM:
        op.code = OP_LAYER_NORM;
        vec_stride_ln = static_cast<int>(packed_size(p, d) / 2);
        op.boff = op.woff + vec_stride_ln;
        op.f0 = d.attr[0];
        break;
      case PONNI_LAYER_SOFTMAX: op.code = OP_SOFTMAX; break;
      case PONNI_LAYER_LOG_SOFTMAX: op.code = OP_LOG_SOFTMAX; break;
      case PONNI_LAYER_MIN_MAX_NORM:
        op.code = OP_MIN_MAX;
        op.f0 = d.attr[0];
        op.f1 = d.attr[1];
        op.f2 = d.attr[2];
        break;
      case PONNI_LAYER_SAVE_STATE: op.code = OP_SAVE; break;
      case PONNI_LAYER_BINOP_ADD: op.code = OP_ADD; break;
      case PONNI_LAYER_BINOP_CONCATENATE:
        op.code = OP_CONCAT;
        op.aux = (d.flags & PONNI_FLAG_CONCAT_AFTER) ? 1 : 0;
        break;
      case PONNI_LAYER_BINOP_PROJECTION_ADD: {
        op.code = OP_PROJ_ADD;
        op.aux = d.n_aux;
        op.boff = static_cast<int32_t>(op.woff + packed_size(p, d) - vec_size(p, d.n_in));
        break;
      }
      case PONNI_LAYER_LOAD_STATE: op.code = OP_LOAD; break;
      case PONNI_LAYER_EXTERNAL:
        op.code = OP_EXTERNAL;
        op.aux = static_cast<int32_t>(d.attr[0]);
        op.boff = d.flags & (PONNI_FLAG_EXT_SAVE | PONNI_FLAG_EXT_BINOP | PONNI_FLAG_EXT_IN_PLACE);
        break;
      case PONNI_LAYER_BINARY:
        op.code = OP_BINARY;
        op.aux = static_cast<int>(d.attr[0]) | ((d.flags & PONNI_FLAG_SAVED_LEFT) ? BIN_SAVED_LEFT : 0) |
                 (d.n_aux == 1 && d.n_out > 1 ? BIN_SAVED_SCALAR : 0) |
                 (d.n_in == 1 && d.n_out > 1 ? BIN_STATE_SCALAR : 0);
        break;
      case PONNI_LAYER_REDUCE:
        op.code = OP_REDUCE;
        op.aux = static_cast<int>(d.attr[0]);
        break;
      case PONNI_LAYER_SELECT: {
        SelectOperands const o = select_operands(d);
        op.code = OP_SELECT;
        op.aux = (o.scalar[0] ? SEL_COND_SCALAR : 0) | (o.scalar[1] ? SEL_A_SCALAR : 0) |
                 (o.scalar[2] ? SEL_B_SCALAR : 0);
        int slots = 0;
        for (int k = 0; k < 3; k++) {
          int code = 0;
          if (o.src[k] == PONNI_SELECT_SLOT) code = ++slots;  // first or second saved operand
          if (o.src[k] == PONNI_SELECT_CONST) code = 3;
          op.aux |= code << (SEL_SRC_BITS * k);
        }
        op.slot = d.slot;
        op.f0 = o.num_slots == 2 ? d.attr[1] : -1.0;
        // Constant operands are packed one after the other.
        op.boff = static_cast<int32_t>(op.woff + (o.num_const == 2 ? vec_size(p, d.n_out) : 0));
        break;
      }
      default: {  // lone pointwise layer
        op.code = OP_POINTWISE;
        op.epi_begin = static_cast<int32_t>(p.steps.size());
        Step s = make_step(d);
        s.off = op.woff;
        p.steps.push_back(s);
        op.epi_count = 1;
        break;
      }
    }
    if (i == 0 && L == 1) {
      op.src = BUF_INPUT;
      op.dst = BUF_OUTPUT;
    } else if (i == 0) {
      // A leading barrier materializes into tmp1; a leading save also fills
      // its slot (ponni_Inference.h:499-514).
      op.src = BUF_INPUT;
      if (is_save(d.kind)) {
        op.dst = BUF_SAVED + d.slot;
        op.aux = 1;  // also copy to tmp1
      } else if (ext_saves(d)) {
        op.dst = BUF_SAVED + d.slot;
        op.boff |= EXT_ALSO_TMP1;
      } else {
        op.dst = BUF_TMP1;
      }
      tmp_max[0] = std::max(tmp_max[0], d.n_out);
      in_tmp1 = true;
    } else if (i < L - 1) {
      // Every built-in barrier declares overwrite_input = true, so the main
      // state keeps its buffer; a save writes its slot instead.  An external
      // layer without overwrite_input writes the other buffer
      // (ponni_Inference.h:518-528).
      op.src = in_tmp1 ? BUF_TMP1 : BUF_TMP2;
      if (is_save(d.kind) || ext_saves(d)) {
        op.dst = BUF_SAVED + d.slot;
      } else if (d.kind == PONNI_LAYER_EXTERNAL && !(d.flags & PONNI_FLAG_EXT_IN_PLACE)) {
        in_tmp1 = !in_tmp1;
        op.dst = in_tmp1 ? BUF_TMP1 : BUF_TMP2;
      } else {
        op.dst = op.src;
      }
      tmp_max[in_tmp1 ? 0 : 1] = std::max(tmp_max[in_tmp1 ? 0 : 1], d.n_out);
    } else {
      op.src = in_tmp1 ? BUF_TMP1 : BUF_TMP2;
      op.dst = BUF_OUTPUT;
    }
    // A load replaces the state with a saved one: it reads the slot and
    // writes where the state lives (or the output).
    if (d.kind == PONNI_LAYER_LOAD_STATE) op.src = BUF_SAVED + d.slot;
    // An op that reads or writes no slot names slot 0, a valid row of the
    // slot table whatever the layer's own (unchecked) slot field holds.
    bool uses_slot = is_save(d.kind) || ext_saves(d) || ext_reads(d) ||
                     (reads_slot(d.kind) && d.kind != PONNI_LAYER_SELECT);
    if (d.kind == PONNI_LAYER_SELECT) uses_slot = select_operands(d).num_slots > 0;
    if (!uses_slot) op.slot = 0;
    p.ops.push_back(op);
    i++;
  }
  p.tmp_features[0] = tmp_max[0];
  p.tmp_features[1] = tmp_max[1];
}

bool mfma_supports(ponni_plan_s const& p) {
  for (auto const& d : p.layers) {
    if (d.kind == PONNI_LAYER_BINOP_CONCATENATE) {
      int const first = (d.flags & PONNI_FLAG_CONCAT_AFTER) ? d.n_in : d.n_out - d.n_in;
      if (first % 16 != 0) return false;  // tile-granular moves only
    }
  }
  return true;
}

// Where each parameter lands in the packed buffer of the plan's path:
// emit(slot, kind, layer, index) names every packed slot that holds
// parameter `index` (master-copy order) of layer `layer`; the slots it never
// names hold zero (padding).
//   SLOT_VALUE  element `slot` of the packed buffer (fp32, or fp64 for F64
//               plans): the value rounded to the plan's type
//   SLOT_HALF   16-bit element `slot` of a 16-bit FUSED buffer: the value's
//               fp16 / bf16 bits (v_mfma_f32_16x16x32 A-fragment order, see
//               fused_f16.h)
//   SLOT_WORD   32-bit word `slot` of a 16-bit FUSED buffer: the value
//               rounded to the plan's 16-bit type, stored as fp32
template <class Emit>
void visit_param_slots(ponni_plan_s const& p, Emit&& emit) {
  bool const half_fused = p.path == PONNI_PATH_FUSED && (p.dtype == PONNI_F16 || p.dtype == PONNI_BF16);
  int const vec_kind = half_fused ? SLOT_WORD : SLOT_VALUE;
  int const L = static_cast<int>(p.layers.size());
  int const W = p.width_class;
  std::vector<int32_t> const in_k = contractions_over_input(p);
  for (int i = 0; i < L; i++) {
    ponni_layer_desc const& d = p.layers[i];
    int64_t const base = p.layer_param_offset[i];
    // (this layer's weights are read by a contraction over the input state)
    bool const k_in = std::find(in_k.begin(), in_k.end(), static_cast<int32_t>(base)) != in_k.end();
    // Dense weights W [K, N] (row k, column n) starting at parameter src0; a
    // transposed source holds W^T [N, K] (generated Dense, "output_input").
    auto dense = [&](int64_t src0, int K, int N, bool transposed) {
      auto idx = [&](int k, int n) { return src0 + (transposed ? int64_t(n) * K + k : int64_t(k) * N + n); };
      if (half_fused) {
        int64_t const hb = 2 * base;  // 16-bit index of the layer's first word
        // v_mfma_f32_16x16x32 A fragment of output tile mo and 32-feature
        // step t: lane l, element j holds W[16(2t + j/4) + 4(l/16) + j%4][16 mo + l%16].
        int const TK = (K + 15) / 16, TN = (N + 15) / 16, TS = (TK + 1) / 2;
        for (int mo = 0; mo < TN; mo++)
          for (int t = 0; t < TS; t++)
            for (int l = 0; l < 64; l++)
              for (int j = 0; j < 8; j++) {
                int const k = 16 * (2 * t + j / 4) + 4 * (l >> 4) + (j & 3);
                int const n = 16 * mo + (l & 15);
                if (k < K && n < N) emit(hb + ((int64_t(mo) * TS + t) * 64 + l) * 8 + j, SLOT_HALF, i, idx(k, n));
              }
      } else if (generic_layout(p)) {
        for (int k = 0; k < K; k++)
          for (int n = 0; n < N; n++) emit(base + int64_t(k) * N + n, SLOT_VALUE, i, idx(k, n));
      } else if (p.path == PONNI_PATH_NARROW) {
        for (int k = 0; k < K; k++)
          for (int n = 0; n < N; n++) emit(base + int64_t(k) * W + n, SLOT_VALUE, i, idx(k, n));
      } else {
        // A fragment of v_mfma_f32_16x16x4f32 for output tile mo and input
        // tile m: lane l, element v holds W[16m + 4(l/16) + v][16mo + l%16]
        // (a contraction over the input state in contraction order, see
        // input_contractions: W[4(4m + v) + l/16][...]).
        // v_mfma_f64_16x16x4f64 returns result row 4e + g in element e of
        // lane group g (fp32: row 4g + e), so fp64 tiles take their A rows in
        // that transposed order and the result lands in the fp32 tile layout.
        bool const rows_t = p.dtype == PONNI_F64;
        int const TK = (K + 15) / 16, TN = (N + 15) / 16;
        for (int mo = 0; mo < TN; mo++)
          for (int m = 0; m < TK; m++)
            for (int l = 0; l < 64; l++)
              for (int v = 0; v < 4; v++) {
                int const k = k_in ? 4 * (4 * m + v) + (l >> 4) : 16 * m + 4 * (l >> 4) + v;
                int const r = l & 15;
                int const n = 16 * mo + (rows_t ? (r & 3) * 4 + (r >> 2) : r);
                if (k < K && n < N) emit(base + ((int64_t(mo) * TK + m) * 64 + l) * 4 + v, SLOT_VALUE, i, idx(k, n));
              }
      }
    };
    // n per-feature values starting at parameter src0, from packed slot base + slot0.
    auto vec = [&](int64_t slot0, int64_t src0, int n) {
      for (int f = 0; f < n; f++) emit(base + slot0 + f, vec_kind, i, src0 + f);
    };
    int64_t const size = packed_size(p, d);
    switch (d.kind) {
      case PONNI_LAYER_MATVEC:
        dense(0, d.n_in, d.n_out, false);
        break;
      case PONNI_LAYER_DENSE:
        dense(0, d.n_in, d.n_out, true);
        if (d.flags & PONNI_FLAG_DENSE_BIAS) vec(size - vec_size(p, d.n_out), int64_t(d.n_out) * d.n_in, d.n_out);
        break;
      case PONNI_LAYER_CONST_BINARY:
      case PONNI_LAYER_BIAS:
        vec(0, 0, d.n_in);
        break;
      case PONNI_LAYER_LAYER_NORM:
        vec(0, 0, d.n_in);
        vec(size / 2, d.n_in, d.n_in);
        break;
      case PONNI_LAYER_BINOP_PROJECTION_ADD:
        dense(0, d.n_aux, d.n_in, false);
        vec(size - vec_size(p, d.n_in), int64_t(d.n_aux) * d.n_in, d.n_in);
        break;
      case PONNI_LAYER_SELECT:
        for (int c = 0; c < select_operands(d).num_const; c++) vec(c * vec_size(p, d.n_out), int64_t(c) * d.n_out, d.n_out);
        break;
      default:
        break;
    }
  }
}

void pack_params(ponni_plan_s const& p, std::vector<double>& out) {
  out.assign(static_cast<size_t>(p.packed_elements), 0.0);
  visit_param_slots(p, [&](int64_t slot, int, int layer, int64_t idx) {
    out[slot] = round_to_dtype(p.params[layer][idx], p.dtype);
  });
}

// Parameters of FUSED fp16 / bf16 plans as 32-bit words: dense blocks hold
// pairs of 16-bit operands in the v_mfma_f32_16x16x32 A-fragment order (see
// fused_f16.h), vectors hold fp32 values already rounded to the operand type.
void pack_words_half(ponni_plan_s const& p, std::vector<uint32_t>& out) {
  out.assign(static_cast<size_t>(p.packed_elements), 0u);
  auto bits16 = [&](double v) -> uint16_t {
    float const f = static_cast<float>(v);
    return p.dtype == PONNI_F16 ? float_to_half_bits(f) : float_to_bf16_bits(f);
  };
  auto* h = reinterpret_cast<uint16_t*>(out.data());
  visit_param_slots(p, [&](int64_t slot, int kind, int layer, int64_t idx) {
    double const v = p.params[layer][idx];
    if (kind == SLOT_HALF) {
      h[slot] = bits16(v);
    } else {
      float const f = static_cast<float>(round_to_dtype(v, p.dtype));
      std::memcpy(&out[slot], &f, 4);
    }
  });
}

int element_size(int dtype) {
  switch (dtype) {
    case PONNI_F64: return 8;
    case PONNI_F16:
    case PONNI_BF16: return 2;
    default: return 4;
  }
}

// Parameters live in the compute type: double for F64, float otherwise.
int param_element_size(ponni_plan_s const& p) { return p.dtype == PONNI_F64 ? 8 : 4; }

#define HIP_TRY(expr)                                                                         \
  do {                                                                                        \
    hipError_t const e_ = (expr);                                                             \
    if (e_ != hipSuccess)                                                                     \
      return fail(PONNI_ERR_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_));       \
  } while (0)

// First parameter (master-copy order) and length of parameter segment `seg`
// of a layer: segment 0 is its first View (Matvec / Dense / projection
// weights, Bias / constant vector, LayerNorm gamma), segment 1 its second
// (LayerNorm beta, projection / Dense bias).  False when it has none.
bool segment_range(ponni_layer_desc const& d, int seg, int64_t& first, int64_t& count) {
  first = 0;
  count = 0;
  switch (d.kind) {
    case PONNI_LAYER_MATVEC: count = seg == 0 ? int64_t(d.n_in) * d.n_out : 0; break;
    case PONNI_LAYER_BIAS:
    case PONNI_LAYER_CONST_BINARY: count = seg == 0 ? d.n_in : 0; break;
    case PONNI_LAYER_LAYER_NORM:
      first = seg == 1 ? d.n_in : 0;
      count = seg <= 1 ? d.n_in : 0;
      break;
    case PONNI_LAYER_BINOP_PROJECTION_ADD:
      first = seg == 1 ? int64_t(d.n_aux) * d.n_in : 0;
      count = seg == 0 ? int64_t(d.n_aux) * d.n_in : seg == 1 ? d.n_in : 0;
      break;
    case PONNI_LAYER_DENSE:
      first = seg == 1 ? int64_t(d.n_out) * d.n_in : 0;
      count = seg == 0 ? int64_t(d.n_out) * d.n_in : (seg == 1 && (d.flags & PONNI_FLAG_DENSE_BIAS)) ? d.n_out : 0;
      break;
    case PONNI_LAYER_SELECT:  // one segment per constant operand, in operand order
      first = int64_t(seg) * d.n_out;
      count = seg >= 0 && seg < select_operands(d).num_const ? d.n_out : 0;
      break;
    default: break;
  }
  return count > 0;
}

double load_host_element(void const* ptr, int dtype, int64_t i) {
  switch (dtype) {
    case PONNI_F64: return static_cast<double const*>(ptr)[i];
    case PONNI_F16: return half_bits_to_float(static_cast<uint16_t const*>(ptr)[i]);
    case PONNI_BF16: return bf16_bits_to_float(static_cast<uint16_t const*>(ptr)[i]);
    default: return static_cast<float const*>(ptr)[i];
  }
}

void store_host_element(void* ptr, int dtype, int64_t i, double v) {
  switch (dtype) {
    case PONNI_F64: static_cast<double*>(ptr)[i] = v; break;
    case PONNI_F16: static_cast<uint16_t*>(ptr)[i] = float_to_half_bits(static_cast<float>(v)); break;
    case PONNI_BF16: static_cast<uint16_t*>(ptr)[i] = float_to_bf16_bits(static_cast<float>(v)); break;
    default: static_cast<float*>(ptr)[i] = static_cast<float>(v); break;
  }
}

// Read shared segment `seg` of layer `i` (device or host array) into `out`.
int read_segment(ponni_plan_s const& p, int i, int seg, std::vector<double>& out) {
  SharedSegment const& s = p.shared[i][seg];
  int64_t first = 0, count = 0;
  segment_range(p.layers[i], seg, first, count);
  out.resize(static_cast<size_t>(count));
  int64_t const rows = count / s.cols;
  if (s.on_device) {
    size_t const es = element_size(s.dtype);
    std::vector<unsigned char> stage(static_cast<size_t>(count) * es);
    HIP_TRY(hipMemcpy2D(stage.data(), es * s.cols, s.ptr, es * s.ld, es * s.cols, rows, hipMemcpyDeviceToHost));
    for (int64_t e = 0; e < count; e++) out[e] = load_host_element(stage.data(), s.dtype, e);
  } else {
    for (int64_t e = 0; e < count; e++) out[e] = load_host_element(s.ptr, s.dtype, (e / s.cols) * s.ld + e % s.cols);
  }
  return PONNI_OK;
}

// Write `values` into shared segment `seg` of layer `i`.
int write_segment(ponni_plan_s const& p, int i, int seg, double const* values) {
  SharedSegment const& s = p.shared[i][seg];
  int64_t first = 0, count = 0;
  segment_range(p.layers[i], seg, first, count);
  int64_t const rows = count / s.cols;
  if (s.on_device) {
    size_t const es = element_size(s.dtype);
    std::vector<unsigned char> stage(static_cast<size_t>(count) * es);
    for (int64_t e = 0; e < count; e++) store_host_element(stage.data(), s.dtype, e, values[e]);
    HIP_TRY(hipMemcpy2D(const_cast<void*>(s.ptr), es * s.ld, stage.data(), es * s.cols, es * s.cols, rows,
                        hipMemcpyHostToDevice));
  } else {
    for (int64_t e = 0; e < count; e++)
      store_host_element(const_cast<void*>(s.ptr), s.dtype, (e / s.cols) * s.ld + e % s.cols, values[e]);
  }
  return PONNI_OK;
}

// Bring the master copy up to date with the shared arrays (device ones only
// when `device`); a change bumps the parameter version, so the GENERIC twins
// are rebuilt, and (host arrays) marks the device copy stale.
int pull_shared(ponni_plan_s& p, bool device) {
  if (p.num_shared_device + p.num_shared_host == 0) return PONNI_OK;
  bool changed = false, host_changed = false;
  std::vector<double> v;
  for (size_t i = 0; i < p.shared.size(); i++)
    for (int seg = 0; seg < 2; seg++) {
      SharedSegment const& s = p.shared[i][seg];
      if (s.ptr == nullptr || (s.on_device && !device)) continue;
      int const st = read_segment(p, static_cast<int>(i), seg, v);
      if (st != PONNI_OK) return st;
      int64_t first = 0, count = 0;
      segment_range(p.layers[i], seg, first, count);
      double* m = p.params[i].data() + first;
      if (!std::equal(v.begin(), v.end(), m)) {
        std::copy(v.begin(), v.end(), m);
        changed = true;
        host_changed = host_changed || !s.on_device;
      }
    }
  if (changed) p.params_version++;
  if (host_changed) p.device_dirty = true;
  return PONNI_OK;
}

// The gather map of the device-shared segments in the plan's packed layout.
int build_gather(ponni_plan_s& p) {
  if (p.d_gather) (void)hipFree(p.d_gather);
  if (p.d_gather_src) (void)hipFree(p.d_gather_src);
  p.d_gather = nullptr;
  p.d_gather_src = nullptr;
  p.gather_count = 0;
  if (p.num_shared_device == 0) return PONNI_OK;
  std::vector<GatherSource> sources;
  std::vector<std::array<int32_t, 2>> table(p.layers.size(), {-1, -1});
  for (size_t i = 0; i < p.shared.size(); i++)
    for (int seg = 0; seg < 2; seg++) {
      SharedSegment const& s = p.shared[i][seg];
      if (s.ptr == nullptr || !s.on_device) continue;
      table[i][seg] = static_cast<int32_t>(sources.size());
      sources.push_back(GatherSource{s.ptr, s.dtype, 0});
    }
  std::vector<GatherEntry> map;
  visit_param_slots(p, [&](int64_t slot, int kind, int layer, int64_t idx) {
    for (int seg = 0; seg < 2; seg++) {
      int64_t first = 0, count = 0;
      if (table[layer][seg] < 0 || !segment_range(p.layers[layer], seg, first, count)) continue;
      if (idx < first || idx >= first + count) continue;
      SharedSegment const& s = p.shared[layer][seg];
      int64_t const e = idx - first;
      map.push_back(GatherEntry{slot, (e / s.cols) * s.ld + e % s.cols, table[layer][seg], kind});
    }
  });
  HIP_TRY(hipMalloc(reinterpret_cast<void**>(&p.d_gather_src), sizeof(GatherSource) * sources.size()));
  HIP_TRY(hipMemcpy(p.d_gather_src, sources.data(), sizeof(GatherSource) * sources.size(), hipMemcpyHostToDevice));
  if (!map.empty()) {
    HIP_TRY(hipMalloc(reinterpret_cast<void**>(&p.d_gather), sizeof(GatherEntry) * map.size()));
    HIP_TRY(hipMemcpy(p.d_gather, map.data(), sizeof(GatherEntry) * map.size(), hipMemcpyHostToDevice));
  }
  p.gather_count = static_cast<int64_t>(map.size());
  return PONNI_OK;
}

int upload(ponni_plan_s& p) {
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  if (p.device >= 0 && p.device != dev)
    return fail(PONNI_ERR_DEVICE, "plan was first used on another device");
  p.device = dev;
  // Parameters may be read by a launch still in flight; the reference's
  // deep_copy fences as well.
  HIP_TRY(hipDeviceSynchronize());
  // The op list, its steps and the slot rows, each sized to the plan.
  if (p.d_ops_count < std::max<size_t>(p.ops.size(), 1)) {
    if (p.d_ops) HIP_TRY(hipFree(p.d_ops));
    p.d_ops = nullptr;
    p.d_ops_count = std::max<size_t>(p.ops.size(), 1);
    HIP_TRY(hipMalloc(reinterpret_cast<void**>(&p.d_ops), sizeof(Op) * p.d_ops_count));
  }
  if (p.d_steps_count < std::max<size_t>(p.steps.size(), 1)) {
    if (p.d_steps) HIP_TRY(hipFree(p.d_steps));
    p.d_steps = nullptr;
    p.d_steps_count = std::max<size_t>(p.steps.size(), 1);
    HIP_TRY(hipMalloc(reinterpret_cast<void**>(&p.d_steps), sizeof(Step) * p.d_steps_count));
  }
  if (p.d_slot_rows == nullptr)
    HIP_TRY(hipMalloc(reinterpret_cast<void**>(&p.d_slot_rows), sizeof(int32_t) * p.slot_rows.size()));
  HIP_TRY(hipMemcpy(p.d_ops, p.ops.data(), sizeof(Op) * p.ops.size(), hipMemcpyHostToDevice));
  if (!p.steps.empty())
    HIP_TRY(hipMemcpy(p.d_steps, p.steps.data(), sizeof(Step) * p.steps.size(), hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(p.d_slot_rows, p.slot_rows.data(), sizeof(int32_t) * p.slot_rows.size(), hipMemcpyHostToDevice));
  std::vector<double> packed;
  std::vector<uint32_t> words;
  bool const half_fused = p.path == PONNI_PATH_FUSED && (p.dtype == PONNI_F16 || p.dtype == PONNI_BF16);
  if (half_fused) pack_words_half(p, words);
  else pack_params(p, packed);
  size_t const count = half_fused ? words.size() : packed.size();
  // Rounded up so vector reads of the last packed block stay inside the allocation.
  size_t const bytes = std::max<size_t>((count * param_element_size(p) + 255) / 256 * 256, 256);
  if (bytes > p.d_params_bytes) {
    if (p.d_params) HIP_TRY(hipFree(p.d_params));
    p.d_params = nullptr;
    HIP_TRY(hipMalloc(&p.d_params, bytes));
    p.d_params_bytes = bytes;
  }
  if (half_fused) {
    if (!words.empty()) HIP_TRY(hipMemcpy(p.d_params, words.data(), words.size() * 4, hipMemcpyHostToDevice));
  } else if (!packed.empty()) {
    if (p.dtype == PONNI_F64) {
      HIP_TRY(hipMemcpy(p.d_params, packed.data(), packed.size() * 8, hipMemcpyHostToDevice));
    } else {
      std::vector<float> f(packed.begin(), packed.end());
      HIP_TRY(hipMemcpy(p.d_params, f.data(), f.size() * 4, hipMemcpyHostToDevice));
    }
  }
  if ((p.path == PONNI_PATH_FUSED || p.narrow_jit) && p.fused_fn == nullptr) {
    std::string error;
    int const st = fused_prepare(p, error);
    if (st != PONNI_OK) return fail(st, error);
  }
  int const st = build_gather(p);
  if (st != PONNI_OK) return st;
  // A GENERIC plan's allocation-free forward carves its state buffers from
  // the fixed per-device scratch; its address is looked up here, where
  // loading the code object that holds it may allocate, so that
  // ponni_forward_no_alloc never does that lookup first.
  if (generic_layout(p)) {
    void* base = nullptr;
    HIP_TRY(static_scratch(dev, &base));
  }
  p.device_dirty = false;
  return PONNI_OK;
}

void release_scratch(ponni_plan_s& p) {
  for (auto& s : p.d_scratch) {
    if (s) (void)hipFree(s);
    s = nullptr;
  }
}

int reallocate_scratch(ponni_plan_s& p, int64_t batch) {
  HIP_TRY(hipDeviceSynchronize());
  release_scratch(p);
  p.capacity = batch;
  if (!generic_layout(p) || batch == 0) return PONNI_OK;
  size_t const es = element_size(p.dtype);
  for (int b = 0; b < 2; b++) {
    if (p.tmp_features[b] > 0)
      HIP_TRY(hipMalloc(&p.d_scratch[b], es * size_t(p.tmp_features[b]) * size_t(batch)));
  }
  if (p.saved_total > 0) HIP_TRY(hipMalloc(&p.d_scratch[2], es * size_t(p.saved_total) * size_t(batch)));
  return PONNI_OK;
}

}  // namespace

namespace ponni_hip {
int set_error(int status, std::string const& message) { return fail(status, message); }
std::vector<int32_t> input_contractions(ponni_plan_s const& p) { return contractions_over_input(p); }
}  // namespace ponni_hip

namespace {

// A double as C++ source that reads back to the same value.
std::string double_literal(double v) {
  if (std::isnan(v)) return "__builtin_nan(\"\")";
  if (std::isinf(v)) return v > 0 ? "__builtin_inf()" : "-__builtin_inf()";
  char b[40];
  std::snprintf(b, sizeof b, "%.17g", v);
  std::string t = b;
  if (t.find_first_of(".eE") == std::string::npos) t += ".0";
  return t;
}

}  // namespace

extern "C" {

const char* ponni_last_error(void) { return g_last_error.c_str(); }

int ponni_abi_version(void) { return PONNI_ABI_VERSION; }

int ponni_plan_create(const ponni_layer_desc* layers, int32_t num_layers, int32_t dtype,
                      int32_t path, ponni_plan* out_plan) {
  g_last_error.clear();
  if (out_plan == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "out_plan is null");
  *out_plan = nullptr;
  if (layers == nullptr || num_layers <= 0) return fail(PONNI_ERR_INVALID_ARGUMENT, "a model needs at least one layer");
  if (dtype < PONNI_F32 || dtype > PONNI_BF16) return fail(PONNI_ERR_INVALID_ARGUMENT, "unknown dtype");
  if (path < PONNI_PATH_AUTO || path > PONNI_PATH_LAYERED) return fail(PONNI_ERR_INVALID_ARGUMENT, "unknown kernel path");
  int const st = validate_chain(layers, num_layers);
  if (st != PONNI_OK) return st;

  auto* p = new (std::nothrow) ponni_plan_s();
  if (p == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "out of host memory");
  p->layers.assign(layers, layers + num_layers);
  p->dtype = dtype;
  p->params.resize(num_layers);
  p->shared.resize(num_layers);
  int max_width = 0;
  for (int i = 0; i < num_layers; i++) {
    auto const& d = layers[i];
    p->params[i].assign(static_cast<size_t>(param_count(d)), 0.0);
    max_width = std::max({max_width, d.n_in, d.n_out,
                          d.kind == PONNI_LAYER_BINOP_PROJECTION_ADD || d.kind == PONNI_LAYER_BINARY ? d.n_aux : 0});
    if (is_save(d.kind) || ext_saves(d)) {
      p->num_slots = std::max(p->num_slots, d.slot + 1);
      if (static_cast<int>(p->saved_features.size()) <= d.slot) p->saved_features.resize(d.slot + 1, 0);
      p->saved_features[d.slot] = std::max(p->saved_features[d.slot], d.n_out);
    }
    if (d.kind == PONNI_LAYER_EXTERNAL) p->external = true;
  }
  p->max_width = max_width;
  set_slot_rows(*p);
  // LayerNorm defaults are gamma = 1, beta = 0 (ponni_LayerNorm.h:39-45).
  for (int i = 0; i < num_layers; i++)
    if (layers[i].kind == PONNI_LAYER_LAYER_NORM)
      for (int f = 0; f < layers[i].n_in; f++) p->params[i][f] = 1.0;

  bool graph_ops = false;
  for (int i = 0; i < num_layers; i++) graph_ops = graph_ops || is_graph_kind(layers[i].kind);
  // Caller-implemented layers run only in the caller's per-sample kernel over
  // the GENERIC op list.
  if (p->external) {
    if (path != PONNI_PATH_AUTO && path != PONNI_PATH_GENERIC) {
      delete p;
      return fail(PONNI_ERR_UNSUPPORTED, "a chain with external (custom) layers runs on the GENERIC op list only");
    }
    path = PONNI_PATH_GENERIC;
  }
  // The interpreted NARROW and MFMA kernels run layer-template chains only;
  // generated NARROW kernels (run-time compilation) also run graph operations
  // and F64.
  int const narrow_w = narrow_width_class(max_width);
  int const narrow = graph_ops ? 0 : narrow_w;
  int const mfma = graph_ops ? 0 : mfma_width_class(dtype, max_width);
  char const* jit_env = std::getenv("PONNI_JIT");
  bool const jit_enabled = jit_env == nullptr || std::strcmp(jit_env, "0") != 0;
  bool const narrow_interp_ok = dtype != PONNI_F64 && narrow > 0 && p->num_slots <= kNarrowMaxSlots;
  bool const narrow_gen_ok = jit_enabled && narrow_w > 0 && !p->external && p->num_slots <= kNarrowJitMaxSlots;
  // Plans only a generated NARROW kernel can run need run-time compilation.
  bool const narrow_ok = narrow_interp_ok || ((graph_ops || dtype == PONNI_F64) && narrow_gen_ok);
  // Between widths 9 and 16 the generated NARROW kernel (scalar FMAs, one
  // lane per sample group) beats FUSED (16-wide MFMA tiles) while the chain
  // does fewer than 10 multiply-adds per byte of input and output; beyond
  // that the matrix cores win (measured on chains of 16-wide layers).
  double macs = 0.0;
  for (int i = 0; i < num_layers; i++) {
    auto const& d = layers[i];
    if (is_dense(d.kind)) macs += double(d.n_in) * d.n_out;
    if (d.kind == PONNI_LAYER_BINOP_PROJECTION_ADD) macs += double(d.n_aux) * d.n_in;
  }
  double const io_bytes = double(layers[0].n_in + layers[num_layers - 1].n_out) * (dtype == PONNI_F32 ? 4 : 2);
  bool const narrow_light = macs < 10.0 * io_bytes;
  // A chain with a dense layer of at least 64 x 64 features is worth running
  // its dense blocks on the matrix cores even with its states in HBM.
  bool layered_pays = false;
  for (int i = 0; i < num_layers; i++)
    layered_pays = layered_pays || (is_dense(layers[i].kind) && layers[i].n_in >= 64 && layers[i].n_out >= 64);
  int chosen = path;
  if (chosen == PONNI_PATH_AUTO) {
    if (narrow_interp_ok && max_width <= 8) chosen = PONNI_PATH_NARROW;
    else if (jit_enabled && narrow_ok && narrow_light) chosen = PONNI_PATH_NARROW;
    else if (jit_enabled && fused_supports(*p)) chosen = PONNI_PATH_FUSED;
    else if (narrow_ok) chosen = PONNI_PATH_NARROW;
    else if (dtype != PONNI_F64 && mfma > 0 && p->num_slots <= kMfmaMaxSlots && mfma_supports(*p)) chosen = PONNI_PATH_MFMA;
    else if (layered_pays) chosen = PONNI_PATH_LAYERED;
    else chosen = PONNI_PATH_GENERIC;
  } else if (chosen == PONNI_PATH_NARROW) {
    if (!narrow_ok) {
      delete p;
      return fail(PONNI_ERR_UNSUPPORTED,
                  "NARROW path needs width <= 16 and a layer-template chain in F32/F16/BF16 with at most 2 saved "
                  "states, or (with run-time compilation) F64 or a generated graph with at most 4");
    }
  } else if (chosen == PONNI_PATH_FUSED) {
    if (!fused_supports(*p)) {
      delete p;
      return fail(PONNI_ERR_UNSUPPORTED, "FUSED path needs width <= " + std::to_string(fused_max_width(dtype)) +
                                             " (fp16 / bf16 1024, fp32 512, fp64 256)");
    }
  } else if (chosen == PONNI_PATH_MFMA) {
    if (dtype == PONNI_F64 || mfma == 0 || p->num_slots > kMfmaMaxSlots || !mfma_supports(*p)) {
      delete p;
      return fail(PONNI_ERR_UNSUPPORTED,
                  "MFMA path needs a layer-template chain in F32/F16/BF16, width <= 256, at most 2 saved states and "
                  "16-aligned concatenation");
    }
  }
  p->path = chosen;
  p->width_class = chosen == PONNI_PATH_NARROW ? narrow_w : chosen == PONNI_PATH_MFMA ? mfma : 0;
  lower(*p);
  if (p->packed_elements > INT32_MAX) {
    delete p;
    return fail(PONNI_ERR_UNSUPPORTED, "the model's parameters exceed 2^31 elements");
  }
  p->narrow_jit = chosen == PONNI_PATH_NARROW && jit_enabled && narrow_jit_supports(*p);
  *out_plan = p;
  return PONNI_OK;
}

void ponni_plan_destroy(ponni_plan plan) {
  if (plan == nullptr) return;
  if (plan->device_twin) ponni_plan_destroy(plan->device_twin);
  if (plan->device >= 0) {
    int cur = 0;
    if (hipGetDevice(&cur) == hipSuccess && cur != plan->device) (void)hipSetDevice(plan->device);
    (void)hipDeviceSynchronize();
    release_scratch(*plan);
    if (plan->d_ops) (void)hipFree(plan->d_ops);
    if (plan->d_steps) (void)hipFree(plan->d_steps);
    if (plan->d_slot_rows) (void)hipFree(plan->d_slot_rows);
    if (plan->d_params) (void)hipFree(plan->d_params);
    if (plan->d_gather) (void)hipFree(plan->d_gather);
    if (plan->d_gather_src) (void)hipFree(plan->d_gather_src);
    if (cur != plan->device) (void)hipSetDevice(cur);
  }
  delete plan;
}

int ponni_plan_get_info(ponni_plan plan, ponni_plan_info* info) {
  if (plan == nullptr || info == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "null plan or info");
  std::memset(info, 0, sizeof(*info));
  info->path = plan->path;
  info->dtype = plan->dtype;
  info->num_layers = static_cast<int32_t>(plan->layers.size());
  info->num_inputs = plan->layers.front().n_in;
  info->num_outputs = plan->layers.back().n_out;
  info->num_fused_dense_blocks = plan->num_fused_blocks;
  info->num_saved_states = plan->num_slots;
  info->tmp1_features = plan->tmp_features[0];
  info->tmp2_features = plan->tmp_features[1];
  for (int s = 0; s < 8 && s < plan->num_slots; s++) info->saved_features[s] = plan->saved_features[s];
  int64_t total = 0;
  for (auto const& v : plan->params) total += static_cast<int64_t>(v.size());
  info->num_parameters = total;
  info->internal_state_capacity = plan->capacity;
  info->max_width = plan->max_width;
  info->width_class = plan->width_class;
  return PONNI_OK;
}

int32_t ponni_plan_saved_state_size(ponni_plan plan, int32_t slot) {
  if (plan == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "plan is null"), -1;
  if (slot < 0 || slot >= plan->num_slots)
    return fail(PONNI_ERR_INVALID_ARGUMENT, "saved-state slot " + std::to_string(slot) + " out of range [0," +
                                                std::to_string(plan->num_slots) + ")"),
           -1;
  return plan->saved_features[slot];
}

int64_t ponni_plan_layer_param_count(ponni_plan plan, int32_t layer) {
  if (plan == nullptr || layer < 0 || layer >= static_cast<int32_t>(plan->layers.size())) {
    fail(PONNI_ERR_INVALID_ARGUMENT, "layer index out of range");
    return -1;
  }
  return static_cast<int64_t>(plan->params[layer].size());
}

int ponni_plan_set_layer_params(ponni_plan plan, int32_t layer, const void* values, int64_t count) {
  if (plan == nullptr || layer < 0 || layer >= static_cast<int32_t>(plan->layers.size()))
    return fail(PONNI_ERR_INVALID_ARGUMENT, "layer index out of range");
  auto& dst = plan->params[layer];
  if (count != static_cast<int64_t>(dst.size()))
    return fail(PONNI_ERR_SHAPE, "layer " + std::to_string(layer) + " expects " + std::to_string(dst.size()) +
                                     " parameters, got " + std::to_string(count));
  if (count > 0 && values == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "values is null");
  if (plan->dtype == PONNI_F64) {
    auto const* v = static_cast<double const*>(values);
    for (int64_t i = 0; i < count; i++) dst[i] = v[i];
  } else {
    auto const* v = static_cast<float const*>(values);
    for (int64_t i = 0; i < count; i++) dst[i] = v[i];
  }
  // A shared segment is the caller's array: the new values go there too.
  for (int seg = 0; seg < 2; seg++) {
    int64_t first = 0, n = 0;
    if (plan->shared[layer][seg].ptr == nullptr || !segment_range(plan->layers[layer], seg, first, n)) continue;
    int const st = write_segment(*plan, layer, seg, dst.data() + first);
    if (st != PONNI_OK) return st;
  }
  plan->device_dirty = true;
  plan->params_version++;
  return PONNI_OK;
}

int ponni_plan_share_layer_params(ponni_plan plan, int32_t layer, int32_t segment, const void* values,
                                  int32_t dtype, int64_t rows, int64_t cols, int64_t ld, int32_t on_device) {
  if (plan == nullptr || layer < 0 || layer >= static_cast<int32_t>(plan->layers.size()))
    return fail(PONNI_ERR_INVALID_ARGUMENT, "layer index out of range");
  int64_t first = 0, count = 0;
  if (segment < 0 || segment > 1 || !segment_range(plan->layers[layer], segment, first, count))
    return fail(PONNI_ERR_INVALID_ARGUMENT, "layer " + std::to_string(layer) + " has no parameter segment " +
                                                std::to_string(segment));
  SharedSegment& s = plan->shared[layer][segment];
  if (s.ptr != nullptr) {
    // The plan keeps the array's current contents when the sharing ends or moves.
    std::vector<double> v;
    int const st = read_segment(*plan, layer, segment, v);
    if (st != PONNI_OK) return st;
    std::copy(v.begin(), v.end(), plan->params[layer].begin() + first);
    (s.on_device ? plan->num_shared_device : plan->num_shared_host)--;
    s = SharedSegment{};
  }
  if (values != nullptr) {
    if (dtype < PONNI_F32 || dtype > PONNI_BF16) return fail(PONNI_ERR_INVALID_ARGUMENT, "unknown dtype");
    if (rows < 0 || cols <= 0 || ld < cols || rows * cols != count)
      return fail(PONNI_ERR_SHAPE, "layer " + std::to_string(layer) + " segment " + std::to_string(segment) +
                                       " holds " + std::to_string(count) + " parameters; the array is [" +
                                       std::to_string(rows) + ", " + std::to_string(cols) + "] with row stride " +
                                       std::to_string(ld));
    s = SharedSegment{values, dtype, on_device ? 1 : 0, cols, ld};
    (s.on_device ? plan->num_shared_device : plan->num_shared_host)++;
    std::vector<double> v;
    int const st = read_segment(*plan, layer, segment, v);
    if (st != PONNI_OK) {
      (s.on_device ? plan->num_shared_device : plan->num_shared_host)--;
      s = SharedSegment{};
      return st;
    }
    std::copy(v.begin(), v.end(), plan->params[layer].begin() + first);
  }
  plan->device_dirty = true;  // rebuilds the packed copy and the gather map
  plan->params_version++;
  return PONNI_OK;
}

int ponni_plan_get_layer_params(ponni_plan plan, int32_t layer, void* values, int64_t count) {
  if (plan == nullptr || layer < 0 || layer >= static_cast<int32_t>(plan->layers.size()))
    return fail(PONNI_ERR_INVALID_ARGUMENT, "layer index out of range");
  int const st = pull_shared(*plan, true);
  if (st != PONNI_OK) return st;
  auto const& src = plan->params[layer];
  if (count != static_cast<int64_t>(src.size()))
    return fail(PONNI_ERR_SHAPE, "layer " + std::to_string(layer) + " holds " + std::to_string(src.size()) +
                                     " parameters, asked for " + std::to_string(count));
  if (count > 0 && values == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "values is null");
  if (plan->dtype == PONNI_F64) {
    auto* v = static_cast<double*>(values);
    for (int64_t i = 0; i < count; i++) v[i] = src[i];
  } else {
    auto* v = static_cast<float*>(values);
    for (int64_t i = 0; i < count; i++) v[i] = static_cast<float>(src[i]);
  }
  return PONNI_OK;
}

int ponni_plan_reallocate_internal_state(ponni_plan plan, int64_t batch) {
  if (plan == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "plan is null");
  if (batch < 0) return fail(PONNI_ERR_SHAPE, "Inference internal-state batch size must be nonnegative");
  return reallocate_scratch(*plan, batch);
}

namespace {

// Bytes of GENERIC state buffers (tmp1, tmp2, saved slots) for `batch`
// columns when carved from one array, each buffer 256-byte aligned; fills
// the byte offset of each (-1: not used).
size_t carved_scratch_bytes(ponni_plan_s const& p, int64_t batch, int64_t (&offset)[3]) {
  size_t const es = element_size(p.dtype);
  size_t total = 0;
  for (int b = 0; b < 3; b++) {
    int const features = b < 2 ? p.tmp_features[b] : p.saved_total;
    offset[b] = -1;
    if (features <= 0) continue;
    offset[b] = static_cast<int64_t>(total);
    total += (es * size_t(features) * size_t(batch) + 255) / 256 * 256;
  }
  return total;
}

// LAYERED: the GENERIC op list in runs, in order on one stream -- each dense
// op one MFMA contraction over the batch (launch_layered_dense), each run of
// other ops one generic_forward launch over that part of the list; the
// timing events, if any, bracket the whole sequence.
hipError_t layered_forward(ponni_plan_s const& p, LaunchArgs a, hipStream_t stream) {
  hipEvent_t const ev_start = a.ev_start, ev_stop = a.ev_stop;
  a.ev_start = a.ev_stop = nullptr;
  if (ev_start != nullptr) {
    hipError_t const e = hipEventRecord(ev_start, stream);
    if (e != hipSuccess) return e;
  }
  int const n = static_cast<int>(p.ops.size());
  for (int o = 0; o < n;) {
    hipError_t e = hipSuccess;
    Op const& op = p.ops[o];
    if (op.code == OP_DENSE) {
      if (op.src >= BUF_SAVED || op.dst >= BUF_SAVED) return hipErrorInvalidValue;  // (never lowered so)
      DenseArgs d{};
      d.x = a.buffers[op.src];
      d.ldx = a.buffer_ld[op.src];
      d.y = a.buffers[op.dst];
      d.ldy = a.buffer_ld[op.dst];
      d.batch = a.batch;
      d.params = a.params;
      d.woff = op.woff;
      d.n_in = op.n_in;
      d.n_out = op.n_out;
      d.epi_begin = op.epi_begin;
      d.epi_count = op.epi_count;
      d.bias_first = (op.aux & DENSE_BIAS_FIRST) ? 1 : 0;
      d.steps = a.steps;
      e = launch_layered_dense(p.dtype, d, stream);
      o++;
    } else {
      int end = o;
      while (end < n && p.ops[end].code != OP_DENSE) end++;
      LaunchArgs run = a;
      run.ops = a.ops + o;
      run.num_ops = end - o;
      e = launch_generic(p.dtype, run, stream);
      o = end;
    }
    if (e != hipSuccess) return e;
  }
  return ev_stop != nullptr ? hipEventRecord(ev_stop, stream) : hipSuccess;
}

int forward_impl(ponni_plan plan, const void* x, int64_t ld_in, void* y, int64_t ld_out, int64_t batch,
                 hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop, bool no_alloc) {
  if (plan == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "plan is null");
  if (plan->external)
    return fail(PONNI_ERR_UNSUPPORTED, "the plan holds external (custom) layers: run it through ponni_plan_device_model");
  if (batch <= 0) return fail(PONNI_ERR_SHAPE, "Inference requires a nonzero batch size");
  if (batch > INT32_MAX) return fail(PONNI_ERR_SHAPE, "batch exceeds INT_MAX");
  if (x == nullptr || y == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "input or output pointer is null");
  if (ld_in < batch || ld_out < batch)
    return fail(PONNI_ERR_SHAPE, "Error: Provided output dimensions do not match the model and input batch");
  bool const was_dirty = plan->device_dirty;
  if (plan->num_shared_host > 0) {
    int const st = pull_shared(*plan, false);
    if (st != PONNI_OK) return st;
  }
  if (plan->device_dirty) {
    if (no_alloc && !was_dirty)
      return fail(PONNI_ERR_INVALID_ARGUMENT,
                  "ponni_forward_no_alloc: a host array shared with the plan (ponni_plan_share_layer_params, "
                  "on_device = 0) changed since the plan was last put on the device; one ponni_forward call, "
                  "which may allocate, uploads the new values (share device arrays to refresh them without one)");
    if (no_alloc)
      return fail(PONNI_ERR_INVALID_ARGUMENT,
                  "ponni_forward_no_alloc: the plan is not on the device yet (its parameters changed or it never "
                  "ran); one ponni_forward or ponni_plan_device_params call, which may allocate, puts it there");
    int const st = upload(*plan);
    if (st != PONNI_OK) return st;
  } else {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev != plan->device) return fail(PONNI_ERR_DEVICE, "plan was first used on another device");
  }
  void* scratch[3] = {};  // tmp1, tmp2, the saved-slot area
  int64_t scratch_ld = 0;
  if (no_alloc) {
    if (generic_layout(*plan)) {
      int64_t offset[3];
      size_t const need = carved_scratch_bytes(*plan, batch, offset);
      if (need > kStaticScratchBytes)
        return fail(PONNI_ERR_SHAPE, "ponni_forward_no_alloc: batch " + std::to_string(batch) + " needs " +
                                         std::to_string(need) + " bytes of state buffers; the fixed scratch holds " +
                                         std::to_string(kStaticScratchBytes) + " bytes (use ponni_forward)");
      void* base = nullptr;
      if (need > 0) HIP_TRY(static_scratch(plan->device, &base));
      for (int b = 0; b < 3; b++)
        if (offset[b] >= 0) scratch[b] = static_cast<char*>(base) + offset[b];
      scratch_ld = batch;
    }
  } else {
    if (generic_layout(*plan) && batch > plan->capacity) {
      int const st = reallocate_scratch(*plan, batch);
      if (st != PONNI_OK) return st;
    } else if (batch > plan->capacity) {
      plan->capacity = batch;  // register paths keep no batch scratch
    }
    for (int b = 0; b < 3; b++) scratch[b] = plan->d_scratch[b];
    scratch_ld = plan->capacity;
  }
  LaunchArgs a{};
  a.ops = plan->d_ops;
  a.num_ops = static_cast<int32_t>(plan->ops.size());
  a.steps = plan->d_steps;
  a.params = plan->d_params;
  a.param_count = plan->packed_elements;
  a.x = x;
  a.ld_x = ld_in;
  a.y = y;
  a.ld_y = ld_out;
  a.batch = batch;
  a.num_inputs = plan->layers.front().n_in;
  a.num_outputs = plan->layers.back().n_out;
  a.buffers[BUF_INPUT] = const_cast<void*>(x);
  a.buffer_ld[BUF_INPUT] = ld_in;
  a.buffers[BUF_OUTPUT] = y;
  a.buffer_ld[BUF_OUTPUT] = ld_out;
  for (int b = 0; b < 3; b++) {
    a.buffers[BUF_TMP1 + b] = scratch[b];
    a.buffer_ld[BUF_TMP1 + b] = scratch_ld;
  }
  a.slot_rows = plan->d_slot_rows;
  a.ev_start = ev_start;
  a.ev_stop = ev_stop;
  hipError_t err = hipSuccess;
  if (plan->gather_count > 0) {
    err = launch_gather(plan->d_gather, plan->gather_count, plan->d_gather_src, plan->d_params, plan->dtype, stream);
    if (err != hipSuccess)
      return fail(PONNI_ERR_DEVICE, std::string("shared-parameter refresh failed: ") + hipGetErrorString(err));
  }
  switch (plan->path) {
    case PONNI_PATH_NARROW:
      err = plan->narrow_jit ? fused_launch(*plan, a, stream)
                             : launch_narrow(plan->dtype, plan->width_class, plan->num_slots, a, stream);
      break;
    case PONNI_PATH_MFMA: err = launch_mfma(plan->dtype, plan->width_class, plan->num_slots, a, stream); break;
    case PONNI_PATH_FUSED: err = fused_launch(*plan, a, stream); break;
    case PONNI_PATH_LAYERED: err = layered_forward(*plan, a, stream); break;
    default: err = launch_generic(plan->dtype, a, stream); break;
  }
  if (err != hipSuccess) return fail(PONNI_ERR_DEVICE, std::string("kernel launch failed: ") + hipGetErrorString(err));
  return PONNI_OK;
}

}  // namespace

int ponni_forward(ponni_plan plan, const void* x, int64_t ld_in, void* y, int64_t ld_out, int64_t batch,
                  hipStream_t stream) {
  return forward_impl(plan, x, ld_in, y, ld_out, batch, stream, nullptr, nullptr, false);
}

int ponni_forward_no_alloc(ponni_plan plan, const void* x, int64_t ld_in, void* y, int64_t ld_out, int64_t batch,
                           hipStream_t stream) {
  return forward_impl(plan, x, ld_in, y, ld_out, batch, stream, nullptr, nullptr, true);
}

int ponni_forward_timed(ponni_plan plan, const void* x, int64_t ld_in, void* y, int64_t ld_out, int64_t batch,
                        hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if (start == nullptr || stop == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "timing events are null");
  return forward_impl(plan, x, ld_in, y, ld_out, batch, stream, start, stop, false);
}

int ponni_forward_steps(ponni_plan plan, const void* const* x, int64_t ld_in, void* const* y, int64_t ld_out,
                        int64_t batch, int32_t sets, int32_t steps, hipStream_t stream, double* ms_per_step) {
  if (x == nullptr || y == nullptr || ms_per_step == nullptr || sets <= 0 || steps <= 0)
    return fail(PONNI_ERR_INVALID_ARGUMENT, "ponni_forward_steps: null arrays or no sets / steps");
  hipEvent_t e0 = nullptr, e1 = nullptr;
  HIP_TRY(hipEventCreate(&e0));
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return fail(PONNI_ERR_DEVICE, "hipEventCreate failed");
  }
  int st = PONNI_OK;
  if (hipEventRecord(e0, stream) != hipSuccess) st = fail(PONNI_ERR_DEVICE, "hipEventRecord failed");
  for (int32_t i = 0; st == PONNI_OK && i < steps; i++)
    st = ponni_forward(plan, x[i % sets], ld_in, y[i % sets], ld_out, batch, stream);
  float ms = 0.0f;
  if (st == PONNI_OK && (hipEventRecord(e1, stream) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                         hipEventElapsedTime(&ms, e0, e1) != hipSuccess))
    st = fail(PONNI_ERR_DEVICE, "timing the forward passes failed");
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (st == PONNI_OK) *ms_per_step = double(ms) / steps;
  return st;
}

int64_t ponni_plan_kernel_source(ponni_plan plan, char* buf, int64_t len) {
  if (plan == nullptr) {
    fail(PONNI_ERR_INVALID_ARGUMENT, "plan is null");
    return -1;
  }
  if (plan->path != PONNI_PATH_FUSED && !plan->narrow_jit) {
    fail(PONNI_ERR_UNSUPPORTED, "only FUSED and generated NARROW plans have a kernel source");
    return -1;
  }
  FusedConfig cfg;
  std::string const src = fused_source(*plan, cfg);
  int64_t const need = static_cast<int64_t>(src.size()) + 1;
  if (buf != nullptr) {
    if (len < need) {
      fail(PONNI_ERR_INVALID_ARGUMENT, "buffer too small for the kernel source");
      return -1;
    }
    std::memcpy(buf, src.c_str(), static_cast<size_t>(need));
  }
  return need;
}

int64_t ponni_plan_program_source(ponni_plan plan, char* buf, int64_t len) {
  if (plan == nullptr) {
    fail(PONNI_ERR_INVALID_ARGUMENT, "plan is null");
    return -1;
  }
  if (plan->dtype != PONNI_F32 && plan->dtype != PONNI_F64) {
    fail(PONNI_ERR_UNSUPPORTED, "per-sample programs run F32 and F64 plans");
    return -1;
  }
  ponni_plan_s const* t = generic_twin(*plan);
  if (t == nullptr) {
    fail(PONNI_ERR_INVALID_ARGUMENT, "out of host memory");
    return -1;
  }
  std::ostringstream o;
  o << "  static constexpr int dtype = " << t->dtype << ";\n";
  o << "  static constexpr int num_ops = " << t->ops.size() << ";\n";
  o << "  static constexpr ponni_hip::Op ops[" << std::max<size_t>(t->ops.size(), 1) << "] = {\n";
  for (Op const& op : t->ops)
    o << "      {" << op.code << ", " << op.n_in << ", " << op.n_out << ", " << op.slot << ", " << op.aux << ", "
      << op.woff << ", " << op.boff << ", " << op.epi_begin << ", " << op.epi_count << ", " << op.src << ", "
      << op.dst << ", " << double_literal(op.f0) << ", " << double_literal(op.f1) << ", " << double_literal(op.f2)
      << "},\n";
  if (t->ops.empty()) o << "      {},\n";
  o << "  };\n";
  o << "  static constexpr ponni_hip::Step steps[" << std::max<size_t>(t->steps.size(), 1) << "] = {\n";
  for (Step const& st : t->steps)
    o << "      {" << st.act << ", " << st.off << ", " << double_literal(st.a) << ", " << double_literal(st.b) << "},\n";
  if (t->steps.empty()) o << "      {},\n";
  o << "  };\n";
  o << "  static constexpr int tmp_features[2] = {" << t->tmp_features[0] << ", " << t->tmp_features[1] << "};\n";
  o << "  static constexpr int num_slots = " << t->num_slots << ";\n";
  o << "  static constexpr int32_t slot_rows[" << t->slot_rows.size() << "] = {";
  for (size_t sl = 0; sl < t->slot_rows.size(); sl++) o << (sl ? ", " : "") << t->slot_rows[sl];
  o << "};\n";
  o << "  static constexpr int saved_total = " << t->saved_total << ";\n";
  std::string const src = o.str();
  int64_t const need = static_cast<int64_t>(src.size()) + 1;
  if (buf != nullptr) {
    if (len < need) {
      fail(PONNI_ERR_INVALID_ARGUMENT, "buffer too small for the program source");
      return -1;
    }
    std::memcpy(buf, src.c_str(), static_cast<size_t>(need));
  }
  return need;
}

int ponni_plan_compile(ponni_plan plan) {
  if (plan == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "plan is null");
  if (plan->path != PONNI_PATH_FUSED && !plan->narrow_jit) return PONNI_OK;
  std::string key, error;
  std::vector<char> code;
  int const st = fused_compile(*plan, key, code, error);
  return st == PONNI_OK ? PONNI_OK : fail(st, error);
}

int ponni_plan_kernel_config(ponni_plan plan, int32_t* threads, int32_t* columns_per_block, int32_t* persistent) {
  if (plan == nullptr || threads == nullptr || columns_per_block == nullptr || persistent == nullptr)
    return fail(PONNI_ERR_INVALID_ARGUMENT, "null argument");
  if (plan->path != PONNI_PATH_FUSED && !plan->narrow_jit)
    return fail(PONNI_ERR_UNSUPPORTED, "only FUSED and generated NARROW plans have a generated kernel");
  std::string key, error;
  std::vector<char> code;
  int const st = fused_compile(*plan, key, code, error);
  if (st != PONNI_OK) return fail(st, error);
  FusedConfig cfg;
  (void)fused_source(*plan, cfg);
  *threads = 64 * cfg.waves;
  *columns_per_block = cfg.columns_per_block;
  *persistent = (cfg.lds_bytes > 0 || cfg.vec_bytes > 0 || cfg.params_in_registers || cfg.persistent_loop) ? 1 : 0;
  return PONNI_OK;
}

int ponni_plan_device_params(ponni_plan plan, const void** params) {
  if (plan == nullptr || params == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "null argument");
  if (plan->device_dirty) {
    int const st = upload(*plan);
    if (st != PONNI_OK) return st;
  }
  *params = plan->d_params;
  return PONNI_OK;
}

}  // extern "C"

namespace ponni_hip {

ponni_plan_s* generic_twin(ponni_plan_s& plan) {
  if (plan.device_twin == nullptr) {
    auto* t = new (std::nothrow) ponni_plan_s();
    if (t == nullptr) return nullptr;
    t->layers = plan.layers;
    t->dtype = plan.dtype;
    t->num_slots = plan.num_slots;
    t->external = plan.external;
    t->max_width = plan.max_width;
    t->saved_features = plan.saved_features;
    t->slot_rows = plan.slot_rows;
    t->saved_total = plan.saved_total;
    t->path = PONNI_PATH_GENERIC;
    t->width_class = 0;
    lower(*t);
    plan.device_twin = t;
  }
  return plan.device_twin;
}

int host_twin(ponni_plan_s& plan, ponni_plan_s*& twin) {
  twin = generic_twin(plan);
  if (twin == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "out of host memory");
  int const st = pull_shared(plan, plan.num_shared_device > 0);
  if (st != PONNI_OK) return st;
  if (plan.host_version != plan.params_version) {
    std::vector<double> packed;
    twin->params = plan.params;
    pack_params(*twin, packed);
    if (twin->dtype == PONNI_F64) twin->host_params_f64 = std::move(packed);
    else twin->host_params_f32.assign(packed.begin(), packed.end());
    plan.host_version = plan.params_version;
  }
  return PONNI_OK;
}

}  // namespace ponni_hip

extern "C" {

int ponni_plan_device_model(ponni_plan plan, ponni_device_model* out) {
  if (plan == nullptr || out == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "null plan or output");
  if (generic_twin(*plan) == nullptr) return fail(PONNI_ERR_INVALID_ARGUMENT, "out of host memory");
  int const pst = pull_shared(*plan, true);
  if (pst != PONNI_OK) return pst;
  ponni_plan_s& t = *plan->device_twin;
  if (plan->twin_version != plan->params_version || t.device_dirty) {
    t.params = plan->params;
    t.device_dirty = true;
    int const st = upload(t);
    if (st != PONNI_OK) return st;
    plan->twin_version = plan->params_version;
  }
  std::memset(out, 0, sizeof(*out));
  out->ops = t.d_ops;
  out->steps = t.d_steps;
  out->params = t.d_params;
  out->num_ops = static_cast<int32_t>(t.ops.size());
  out->dtype = t.dtype;
  out->num_inputs = t.layers.front().n_in;
  out->num_outputs = t.layers.back().n_out;
  out->max_width = t.max_width;
  out->tmp_features[0] = t.tmp_features[0];
  out->tmp_features[1] = t.tmp_features[1];
  out->num_slots = t.num_slots;
  out->saved_total = t.saved_total;
  out->slot_rows = t.d_slot_rows;
  return PONNI_OK;
}

int ponni_fill_synthetic(void* x, int32_t dtype, int64_t n, uint64_t seed, uint64_t tag, int32_t dist, double a,
                         double b, hipStream_t stream) {
  if (x == nullptr && n > 0) return fail(PONNI_ERR_INVALID_ARGUMENT, "buffer is null");
  if (n < 0) return fail(PONNI_ERR_INVALID_ARGUMENT, "negative element count");
  if (dtype < PONNI_F32 || dtype > PONNI_BF16) return fail(PONNI_ERR_INVALID_ARGUMENT, "unknown dtype");
  if (dist != PONNI_DIST_UNIFORM && dist != PONNI_DIST_NORMAL) return fail(PONNI_ERR_INVALID_ARGUMENT, "unknown distribution");
  if (n == 0) return PONNI_OK;
  hipError_t const err = launch_fill(x, dtype, n, seed, tag, dist, a, b, stream);
  if (err != hipSuccess) return fail(PONNI_ERR_DEVICE, std::string("fill launch failed: ") + hipGetErrorString(err));
  return PONNI_OK;
}

}  // extern "C"
