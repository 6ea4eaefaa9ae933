// FUSED path: per-plan kernel specialization.
//
// The reference instantiates one executor per model at C++ compile time
// (traverse_mixed_batch_parallel, src/ponni_Inference.h:453-555, and the
// generated infer_batch of kokkos_nn/emitter.py:1537-1550).  Here the plan's
// lowered op list is turned into HIP source that calls the tile library of
// fused_f32.h with every width a compile-time constant; hipRTC compiles it for
// gfx950 once per distinct source (in-process and on-disk cache), and the
// module is launched like any other kernel.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>
#include <climits>
#include <dlfcn.h>
#include <link.h>
#include <sys/stat.h>
#include <unistd.h>

#include "fused.h"

namespace ponni_hip {

// Embedded header texts (generated at build time from csrc/*.h).
extern char const* const kJitHeaderNames[];
extern char const* const kJitHeaderTexts[];
extern int const kJitHeaderCount;

namespace {

int tiles(int n) { return (n + 15) / 16; }

std::string flit(float v) {
  char buf[64];
  std::snprintf(buf, sizeof(buf), "%a", static_cast<double>(v));
  return std::string(buf) + "f";
}

// A double literal, exact (F64 plans keep every attribute in double).
std::string dlit(double v) {
  char buf[64];
  std::snprintf(buf, sizeof(buf), "%a", v);
  return buf;
}

// Steps that keep a zero padding row at zero (padded parameter entries are 0).
bool zero_at_zero(int act) {
  switch (act) {
    case ACT_BIAS:
    case ACT_RELU:
    case ACT_LEAKY_RELU:
    case ACT_ELU:
    case ACT_SELU:
    case ACT_GELU_ERF:
    case ACT_GELU_TANH:
    case ACT_SILU:
    case ACT_TANH:
    case ACT_HARD_SWISH:
    case ACT_MISH:
    case ACT_ABS:
    case ACT_NEG:
    case ACT_SQRT:
    case ACT_SOFTSIGN:
    case ACT_CELU:
    case ACT_ERF:
    case ACT_SELU_AG:
    case ACT_MUL_C:
    case ACT_ASIN:
    case ACT_ASINH:
    case ACT_ATAN:
    case ACT_ATANH:
    case ACT_CEIL:
    case ACT_FLOOR:
    case ACT_SIN:
    case ACT_SINH:
    case ACT_TAN:
    case ACT_ROUND:
    case ACT_SIGN:
    case ACT_IS_NAN:
    case ACT_IS_INF:
    case ACT_NONZERO:
      return true;
    case ACT_THRESHOLDED_RELU:
      return true;  // 0 > a ? 0 : 0
    default:
      return false;
  }
}

// Binary operation (ponni_binary_op) on operand expressions l and r.
std::string binary_expr(int op, std::string const& l = "x", std::string const& r = "y") {
  switch (op) {
    case PONNI_BINARY_ADD: return l + " + " + r;
    case PONNI_BINARY_SUB: return l + " - " + r;
    case PONNI_BINARY_MUL: return l + " * " + r;
    case PONNI_BINARY_DIV: return l + " / " + r;
    case PONNI_BINARY_MIN: return l + " < " + r + " ? " + l + " : " + r;
    case PONNI_BINARY_MAX: return l + " > " + r + " ? " + l + " : " + r;
    case PONNI_BINARY_POW: return "d_pow(" + l + ", " + r + ")";
    default: return "apply_binary(" + std::to_string(op) + ", " + l + ", " + r + ")";
  }
}

// f(v, c) of a step with a constant vector operand.
std::string const_expr(Step const& st) {
  if (st.act == ACT_CBIN) return st.b != 0 ? binary_expr(static_cast<int>(st.a), "c", "v")
                                           : binary_expr(static_cast<int>(st.a), "v", "c");
  switch (st.act) {
    case ACT_BIAS: return "v + c";
    case ACT_SUB_C: return "v - c";
    case ACT_RSUB_C: return "c - v";
    case ACT_MUL_C: return "v * c";
    case ACT_DIV_C: return "v / c";
    case ACT_RDIV_C: return "c / v";
    case ACT_MIN_C: return "v < c ? v : c";
    case ACT_RMIN_C: return "c < v ? c : v";
    case ACT_MAX_C: return "v > c ? v : c";
    case ACT_RMAX_C: return "c > v ? c : v";
    case ACT_POW_C: return "d_pow(v, c)";
    default: return "d_pow(c, v)";
  }
}

// The step's activation on v (float, or double when dbl), in the reference
// formulas of pointwise.h.
std::string act_expr(Step const& s, bool dbl = false) {
  auto lit = [&](double v) { return dbl ? dlit(v) : flit(static_cast<float>(v)); };
  switch (s.act) {
    case ACT_RELU: return "act_relu(v)";
    case ACT_LEAKY_RELU: return "act_leaky_relu(v, " + lit(s.a) + ")";
    case ACT_ELU: return "act_elu(v, " + lit(s.a) + ")";
    case ACT_SELU: return "act_selu(v)";
    case ACT_GELU_ERF: return "act_gelu_erf(v)";
    case ACT_GELU_TANH: return "act_gelu_tanh(v)";
    case ACT_SILU: return "act_silu(v)";
    case ACT_SIGMOID: return "act_sigmoid(v)";
    case ACT_TANH: return "act_tanh(v)";
    case ACT_SOFTPLUS: return "act_softplus(v, " + lit(s.a) + ")";
    case ACT_HARD_SIGMOID: return "act_hard_sigmoid(v, " + lit(s.a) + ", " + lit(s.b) + ")";
    case ACT_HARD_SWISH: return "act_hard_swish(v)";
    case ACT_MISH: return "act_mish(v)";
    case ACT_ABS: return "d_abs(v)";
    case ACT_NEG: return "-v";
    case ACT_EXP: return "d_exp(v)";
    case ACT_LOG: return "d_log(v)";
    case ACT_SQRT: return "d_sqrt(v)";
    case ACT_RECIPROCAL: return "1 / v";
    case ACT_SOFTSIGN: return "act_softsign(v)";
    case ACT_CELU: return "act_celu(v, " + lit(s.a) + ")";
    case ACT_THRESHOLDED_RELU: return "act_thresholded_relu(v, " + lit(s.a) + ")";
    case ACT_ERF: return "d_erf(v)";
    case ACT_SELU_AG: return "act_selu_ag(v, " + lit(s.a) + ", " + lit(s.b) + ")";
    case ACT_ACOS: return "d_acos(v)";
    case ACT_ACOSH: return "d_acosh(v)";
    case ACT_ASIN: return "d_asin(v)";
    case ACT_ASINH: return "d_asinh(v)";
    case ACT_ATAN: return "d_atan(v)";
    case ACT_ATANH: return "d_atanh(v)";
    case ACT_CEIL: return "d_ceil(v)";
    case ACT_COS: return "d_cos(v)";
    case ACT_COSH: return "d_cosh(v)";
    case ACT_FLOOR: return "d_floor(v)";
    case ACT_SIN: return "d_sin(v)";
    case ACT_SINH: return "d_sinh(v)";
    case ACT_TAN: return "d_tan(v)";
    case ACT_ROUND: return "d_round(v)";
    case ACT_SIGN: return "act_sign(v)";
    case ACT_IS_NAN: return "act_is_nan(v)";
    case ACT_IS_INF: return "act_is_inf(v, " + lit(s.a) + ", " + lit(s.b) + ")";
    case ACT_NOT: return "act_not(v)";
    case ACT_NONZERO: return "act_nonzero(v)";
    default: return "v";
  }
}

// The generated kernels' form: the logistic family on the hardware 2^x and 1/x.
std::string act_fast_expr(Step const& s) {
  switch (s.act) {
    case ACT_TANH: return "act_tanh_fast(v)";
    case ACT_SIGMOID: return "act_sigmoid_fast(v)";
    case ACT_SILU: return "act_silu_fast(v)";
    case ACT_GELU_TANH: return "act_gelu_tanh_fast(v)";
    default: return act_expr(s);
  }
}

uint64_t fnv(std::string const& s) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (unsigned char ch : s) {
    h ^= ch;
    h *= 0x100000001b3ull;
  }
  return h;
}

struct Module {
  hipModule_t module = nullptr;
  hipFunction_t fn = nullptr;
  int blocks_per_cu = 0;
};

std::mutex g_mutex;
std::map<std::pair<int, std::string>, std::shared_ptr<Module>> g_modules;  // (device, key)

std::string cache_dir() {
  if (char const* d = std::getenv("PONNI_JIT_CACHE")) return d;
  if (char const* d = std::getenv("XDG_CACHE_HOME")) return std::string(d) + "/ponni_hip";
  if (char const* d = std::getenv("HOME")) return std::string(d) + "/.cache/ponni_hip";
  return "";
}

// fp32 / fp64 plans compile with -ffp-contract=on: multiply-adds fuse within
// one expression (a dot product's terms) but not across statements, so a
// layer's state is rounded before the next layer reads it, as the reference
// materializes it.  (Fused across layers, Mish's last product entered
// MinMaxNorm's x - min unrounded and a sub-ulp difference was scaled by
// 1 / (max - min).)  16-bit plans round their state to the 16-bit type at
// every op or block boundary (an epilogue fused into its dense block stays
// in fp32 until that rounding, within an fp32 ulp of the unfused
// evaluation), which already stops that, and keep the default.
std::vector<char const*> jit_options(bool contract) {
  std::vector<char const*> o{"--offload-arch=gfx950", "-O3", "-std=c++17"};
  if (contract) o.push_back("-ffp-contract=on");
  for (char const* x : {"-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"}) o.push_back(x);
  return o;
}

bool contract_on(ponni_plan_s const& p) { return p.dtype == PONNI_F32 || p.dtype == PONNI_F64; }

bool compile(std::string const& source, bool contract, std::vector<char>& code, std::string& log) {
  hiprtcProgram prog = nullptr;
  if (hiprtcCreateProgram(&prog, source.c_str(), "ponni_fused.hip", kJitHeaderCount, kJitHeaderTexts,
                          kJitHeaderNames) != HIPRTC_SUCCESS) {
    log = "hiprtcCreateProgram failed";
    return false;
  }
  std::vector<char const*> const opts = jit_options(contract);
  hiprtcResult const r = hiprtcCompileProgram(prog, int(opts.size()), opts.data());
  size_t n = 0;
  hiprtcGetProgramLogSize(prog, &n);
  log.assign(n, '\0');
  if (n) hiprtcGetProgramLog(prog, &log[0]);
  if (r != HIPRTC_SUCCESS) {
    hiprtcDestroyProgram(&prog);
    return false;
  }
  hiprtcGetCodeSize(prog, &n);
  code.resize(n);
  hiprtcGetCode(prog, code.data());
  hiprtcDestroyProgram(&prog);
  return true;
}

}  // namespace

// Can the FUSED generator express this chain?
// Widest state a FUSED kernel keeps in registers: 16-bit states up to 1024
// features, fp32 up to 512 and fp64 up to 256 (one 16-column tile per wave
// beyond 256 features).
int fused_max_width(int dtype) {
  return dtype == PONNI_F64 ? 256 : (dtype == PONNI_F16 || dtype == PONNI_BF16) ? 1024 : 512;
}

bool fused_supports(ponni_plan_s const& p) { return p.max_width <= fused_max_width(p.dtype); }

// 16-column tiles per wave: two, one for plans wider than 256 features
// (a 16-bit 512-feature chain with two spills 72 registers at one wave per
// SIMD; with one it runs spill-free).
int fused_nt(ponni_plan_s const& p) { return p.max_width > 256 ? 1 : 2; }

// Generate the HIP source of the plan's kernel.  Offsets are those of the
// MFMA packing (plan.cpp, pack_params).
// Kernel symbol: ponni_fused_<in>x..x<out>_<hash of the op list>, so traces name the model.
std::string fused_kernel_name(ponni_plan_s const& p) {
  std::string sig((char const*)p.ops.data(), p.ops.size() * sizeof(Op));
  sig.append((char const*)p.steps.data(), p.steps.size() * sizeof(Step));
  std::string widths = std::to_string(p.layers.front().n_in);
  for (Op const& op : p.ops)
    if (op.code == OP_DENSE) widths += "x" + std::to_string(op.n_out);
  char buf[16];
  std::snprintf(buf, sizeof(buf), "%08x", static_cast<unsigned>(fnv(sig) & 0xffffffffu));
  return std::string(p.path == PONNI_PATH_NARROW ? "ponni_narrow_" : "ponni_fused_") + widths + "_" + buf;
}

std::string narrow_source_of(ponni_plan_s const& p, FusedConfig& cfg);

namespace {
std::string fused_source_once(ponni_plan_s const& p, FusedConfig& cfg, bool allow_vec_staging);
}  // namespace

// A staged 16-bit plan whose per-feature vectors would not fit next to the
// staging slots and input rows keeps them in global memory (L2).
std::string fused_source(ponni_plan_s const& p, FusedConfig& cfg) {
  FusedConfig first = cfg;
  std::string src = fused_source_once(p, first, true);
  if (first.lds_total > kFusedLdsBytes && first.vec_bytes > 0) return fused_source_once(p, cfg, false);
  cfg = first;
  return src;
}

namespace {
std::string fused_source_once(ponni_plan_s const& p, FusedConfig& cfg, bool allow_vec_staging) {
  if (p.path == PONNI_PATH_NARROW) return narrow_source_of(p, cfg);
  bool const half = p.dtype == PONNI_F16 || p.dtype == PONNI_BF16;
  bool const dbl = p.dtype == PONNI_F64;  // fp64 tiles (v_mfma_f64_16x16x4f64)
  std::string const E = p.dtype == PONNI_BF16 ? "__bf16" : "_Float16";
  // Scalar and 4-vector types of the fp32 / fp64 tiles in emitted code (the
  // 16-bit path's fp32 accumulators stay float).
  std::string const F = half ? "float" : "real", F4 = half ? "floatx4" : "realx4";
  int const es = dbl ? 8 : 4;  // packed parameter element bytes
  auto lit = [&](double v) { return dbl ? dlit(v) : flit(static_cast<float>(v)); };
  // 16-column tiles per wave: two (one beyond 256 features).  16-bit plans
  // run two waves per SIMD with A fragments staged through LDS (fused_f16.h
  // dense_hs), or one when the widest layer's two states do not fit in
  // half the registers.
  int const NT = fused_nt(p);
  // 16-bit plans: two waves per SIMD (one eight-wave workgroup per CU), the
  // compile permitting (fused_compile).
  int const half_wps = 2;
  int64_t const param_bytes = (p.packed_elements * es + 31) / 32 * 32;
  cfg.lds_bytes = !half && param_bytes <= kFusedLdsParamBytes ? static_cast<int>(param_bytes) : 0;
  cfg.waves = 4;
  // Register budget.  A live tile holds 8 registers per lane (fp32 with 2
  // column tiles, or 16-bit with 4); a dense op holds its input, its output
  // and its A-fragment ring.  Parameters small enough to live in registers
  // next to that state are loaded once per wave and reused for every tile.
  int worst = 0, worst_saved_regs = 0;
  int const tr = (dbl ? 8 : 4) * NT;  // registers per lane of one fp32 / fp64 tile
  {
    int cur = tiles(p.layers.front().n_in);
    std::map<int, int> slots;
    for (Op const& op : p.ops) {
      int saved_regs = 0;
      for (auto const& kv : slots) saved_regs += kv.second * tr;
      worst_saved_regs = std::max(worst_saved_regs, saved_regs);
      int need = cur * tr;
      switch (op.code) {
        case OP_DENSE:
          need = (tiles(op.n_in) + tiles(op.n_out)) * tr + (half ? 16 + 2 * NT * 4 : tiles(op.n_in) * tr / 2);
          cur = tiles(op.n_out);
          break;
        case OP_PROJ_ADD: need = (cur + 2 * tiles(op.n_out)) * tr + tiles(op.aux) * tr / 2; break;
        case OP_CONCAT: need = 2 * tiles(op.n_out) * tr; cur = tiles(op.n_out); break;
        case OP_SAVE: slots[op.slot] = cur; break;
        case OP_LOAD: cur = tiles(op.n_out); need = cur * tr; break;
        case OP_BINARY: need = (cur + 2 * tiles(op.n_out)) * (half ? 16 : tr); cur = tiles(op.n_out); break;
        case OP_SELECT: need = (cur + 4 * tiles(op.n_out)) * (half ? 16 : tr); cur = tiles(op.n_out); break;
        case OP_REDUCE: need = cur * (half ? 16 : tr); cur = 1; break;
        default: need = half ? cur * 16 : cur * tr; break;  // 16-bit states widen to fp32 for barriers
      }
      worst = std::max(worst, need + saved_regs);
    }
  }
  int const overhead = 32;
  int64_t const param_regs = (p.packed_elements + 63) / 64;
  cfg.params_in_registers = !half && !dbl && worst + overhead + param_regs <= 256;
  int regs = worst + overhead + (cfg.params_in_registers ? static_cast<int>(param_regs) : 0);
  if (cfg.params_in_registers) cfg.lds_bytes = 0;
  // Saved residuals move to LDS when that is what it takes to run two waves
  // per SIMD (so one wave's VALU epilogue overlaps another's MFMAs).
  if (!half) {
    int saved_tiles = 0;
    for (int s = 0; s < p.num_slots; s++) saved_tiles += tiles(p.saved_features[s]);
    int const saved_bytes = saved_tiles * NT * 64 * 4 * es * 4;  // per workgroup (4 waves)
    if (regs + 32 > 256 && worst_saved_regs > 0 && regs - worst_saved_regs <= 224 &&
        cfg.lds_bytes + saved_bytes <= 80 * 1024) {
      cfg.saved_in_lds = true;
      regs -= worst_saved_regs;
    }
  }
  cfg.waves_per_simd = regs <= 128 ? 4 : regs <= 168 ? 3 : regs <= 256 ? 2 : 1;
  if (half) cfg.waves_per_simd = half_wps;
  if (p.fused_wps > 0) cfg.waves_per_simd = p.fused_wps;  // measured by fused_compile

  // Waves per workgroup: LDS-staged parameters are copied once per
  // workgroup, so when copies would cap the resident workgroups below the
  // register-limited occupancy, fewer and larger workgroups share one copy.
  {
    int saved_per_wave = 0;  // bytes of LDS-resident saved states per wave
    if (cfg.saved_in_lds)
      for (int s = 0; s < p.num_slots; s++) saved_per_wave += tiles(p.saved_features[s]) * NT * 64 * 4 * es;
    int const target = 4 * cfg.waves_per_simd;  // waves per CU the registers allow
    int best = 0;
    for (int w = 4; w <= 16; w += 4) {
      int const per_block_lds = cfg.lds_bytes + w * saved_per_wave;
      if (per_block_lds > 160 * 1024) break;
      int const by_lds = per_block_lds > 0 ? (160 * 1024) / per_block_lds : 1 << 20;
      int const blocks = std::min(by_lds, target / w);
      if (blocks * w > best) {
        best = blocks * w;
        cfg.waves = w;
      }
    }
  }
  // A workgroup of 16-bit plans is one wave per SIMD per occupancy level: its
  // waves share the staged A fragments and the activation table.
  if (half) cfg.waves = 4 * std::min(cfg.waves_per_simd, half_wps);
  cfg.columns_per_block = cfg.waves * 16 * NT;

  std::ostringstream o;
  std::string const IO = half ? E : dbl ? std::string("double") : std::string("float");
  o << "// generated by libponni_hip for one plan\n";
  // fp32 plans whose parameters sit in LDS or registers keep each dense
  // tile's epilogue among the next tile's MFMAs (fused_f32.h dense_ep; c2
  // and c5 2.8 / 3.5 % faster).  Plans streaming parameters from L2 keep the
  // compiler's order: measured neutral at their occupancy (c3), and the
  // registers it frees would move c3 to two waves per SIMD, 8 % slower.
  int const epi_interleave = (!half && !dbl && (cfg.lds_bytes > 0 || cfg.params_in_registers)) ? 16 : 0;

  if (dbl) o << "#define PONNI_REAL double\n";
  if (NT != 2) o << "#define PONNI_NT " << NT << "\n";
  // One column tile per wave at two waves per SIMD: A fragments read two
  // steps ahead (fused_f16.h kFragPipe; 64x512x512x64 3.28 against 3.38 ms,
  // 320 / 384 features 5-7 % faster; at one wave per SIMD, and with two
  // column tiles per wave (c4), reading ahead measured slower).
  if (half && NT == 1 && cfg.waves_per_simd >= 2) o << "#define PONNI_PIPE 2\n";
  o << "#include \"" << (half ? "fused_f16.h" : "fused_f32.h") << "\"\n";
  o << "using namespace ponni_hip;\nusing namespace ponni_hip::fused;\n";
  if (half) o << "typedef " << E << " E;\n";
  o << "extern \"C\" __global__ __launch_bounds__(" << 64 * cfg.waves << ", " << cfg.waves_per_simd << ") void "
    << fused_kernel_name(p)
    << "(" << F << " const* __restrict__ gparams, " << IO << " const* __restrict__ x, int64_t ldx, " << IO
    << "* __restrict__ y, int64_t ldy, int64_t batch) {\n";
  if (cfg.lds_bytes > 0) {
    o << "  __shared__ " << F4 << " lds_p[" << cfg.lds_bytes / (4 * es) << "];\n";
    o << "  stage(lds_p, gparams, " << cfg.lds_bytes / es << ");\n";
    o << "  " << F << " const* __restrict__ P0 = reinterpret_cast<" << F << " const*>(lds_p);\n";
  } else {
    o << "  " << F << " const* __restrict__ P0 = gparams;\n";
  }
  // 16-bit plans: dense layers in program order, and the chunks their A
  // fragments are staged in (fused_f16.h Stage): per layer, as many output
  // tiles per chunk as fill a 32-fragment slot, the last chunk partial.
  struct DenseRef {
    int woff, ts, to;
  };
  std::vector<DenseRef> dense_seq;
  for (Op const& op : p.ops)
    if (op.code == OP_DENSE) dense_seq.push_back(DenseRef{op.woff, (tiles(op.n_in) + 1) / 2, tiles(op.n_out)});
  int const slot_frags = 32, slots = 3;
  if (half && !dense_seq.empty()) {
    std::ostringstream tab;
    int chunks = 0;
    for (DenseRef const& d : dense_seq) {
      int const ct = slot_frags / d.ts;
      for (int t0 = 0; t0 < d.to; t0 += ct, chunks++)
        tab << (chunks ? ", " : "") << d.woff + t0 * d.ts * 256 << ", " << std::min(ct, d.to - t0) * d.ts;
    }
    o << "  __shared__ Vec<E>::x8 a_slots[kSlots * kSlotFrags * 64];\n";
    o << "  static constexpr int chunk_tab[" << 2 * chunks << "] = {" << tab.str() << "};\n";
    o << "  Stage<E> st{a_slots, reinterpret_cast<E const*>(gparams), chunk_tab, " << chunks << ", 0};\n";
    o << "  stage_begin<" << cfg.waves << ">(st);\n";
    cfg.persistent_loop = true;
  }
  size_t dense_index = 0;
  std::map<int, int> slot_off;  // slot -> 4-vector offset in the wave's LDS region
  if (cfg.saved_in_lds) {
    int off = 0;
    for (int sl = 0; sl < p.num_slots; sl++)
      if (p.saved_features[sl] > 0) {
        slot_off[sl] = off;
        off += tiles(p.saved_features[sl]) * NT * 64;
      }
    o << "  __shared__ " << F4 << " lds_saved[" << cfg.waves << "][" << off << "];\n";
    o << "  " << F4 << "* __restrict__ SV = lds_saved[threadIdx.x >> 6];\n";
  }
  // Per-feature vectors (biases, LayerNorm gamma / beta, constant operands)
  // of plans whose parameters stream from L2 are staged into LDS once per
  // workgroup, so the tile loop issues no global load besides its A
  // fragments (a late global load would wait behind them: vmcnt is in order).
  // (Measured: c4 unchanged, c3 slower as a persistent fp32 kernel, so only
  // 16-bit plans, which are persistent anyway, stage them by default.)
  bool const stage_vecs = allow_vec_staging && half && cfg.lds_bytes == 0 && !cfg.params_in_registers;
  std::map<int, std::pair<int, int>> vec_lds;  // packed offset -> (LDS offset, length)
  int vec_total = 0;
  auto vec = [&](int off, int n) -> std::string {
    if (!stage_vecs) return "P + " + std::to_string(off);
    int const len = (n + 15) / 16 * 16;
    auto it = vec_lds.find(off);
    if (it == vec_lds.end()) {
      it = vec_lds.emplace(off, std::make_pair(vec_total, len)).first;
      vec_total += len;
    } else if (it->second.second < len) {
      it->second.second = len;  // never happens for a consistent plan; keep the longest
    }
    return "VP + " + std::to_string(it->second.first);
  };
  // Contractions over the input state in contraction order (plan.cpp
  // input_contractions): ", KS" with the steps that hold input features.
  std::vector<int32_t> const in_k = half ? std::vector<int32_t>() : input_contractions(p);
  auto k_steps = [&](int32_t woff, int n_in) -> std::string {
    if (std::find(in_k.begin(), in_k.end(), woff) == in_k.end()) return "";
    return ", " + std::to_string((n_in + 3) / 4);
  };
  std::ostringstream head;
  head << o.str();
  o.str("");
  o << "  Lane L;\n  L.lane = threadIdx.x & 63;\n  L.g = L.lane >> 4;\n  L.c = L.lane & 15;\n  L.batch = batch;\n";
  o << "  int64_t const tiles = (batch + " << cfg.columns_per_block - 1 << ") / " << cfg.columns_per_block << ";\n";
  // 16-bit plans request each tile's input rows into LDS one tile ahead
  // (fused_f16.h prefetch_rows_lds16) when the buffer fits next to the staged
  // A fragments (3 slots of 32 KB) and vectors.
  int const n_in0 = p.layers.front().n_in;
  int const in_rows_elems = tiles(n_in0) * 16 * 16 * NT;  // per wave, row-major 16-bit
  int const in_dma_bytes = cfg.waves * in_rows_elems * 2;
  int const stage_bytes = half && !dense_seq.empty() ? slots * slot_frags * 1024 : 0;
  bool const in_dma = half && NT % 2 == 0 && in_dma_bytes <= 64 * 1024 &&
                      in_dma_bytes + stage_bytes + 16 * 1024 <= kFusedLdsBytes;
  std::string const WCOLS = std::to_string(16 * NT), NW = std::to_string(cfg.waves);
  // The next tile's rows are requested inside the second dense layer, right
  // after its first chunk's weight loads (fused_f16.h dense_hs hook): waits
  // for weight chunks (vmcnt counts in issue order) then never wait for
  // them, the next one a chunk later.  With one dense layer: after this
  // tile's rows are read.
  int const hook_dense = half && in_dma && dense_seq.size() >= 2 ? 1 : -1;
  std::string const prefetch_next = "if (pre_next) prefetch_rows_lds16<" + std::to_string(n_in0) + ", " +
                                    std::to_string(NT) + ">(x, ldx, Ln, in_buf[wave_id()]);";
  // The last op, a dense layer whose epilogue is its bias (the seed) and
  // activations without parameters, runs transposed and writes 8-byte runs
  // of output rows (fused_f16.h store_rows_ht).
  bool out_transposed = false;
  if (half && !p.ops.empty() && p.ops.back().code == OP_DENSE) {
    Op const& op = p.ops.back();
    bool const lead = op.epi_count > 0 && p.steps[op.epi_begin].act == ACT_BIAS;
    out_transposed = true;
    for (int s = lead ? 1 : 0; s < op.epi_count; s++) {
      int const a = p.steps[op.epi_begin + s].act;
      if (a == ACT_BIAS || act_has_param(a)) out_transposed = false;
    }
  }
  if (out_transposed)
    o << "  bool const yvec = ((reinterpret_cast<uint64_t>(y) | uint64_t(ldy) * 2) & 7) == 0;\n";
  if (in_dma) {
    o << "  __shared__ unsigned short in_buf[" << cfg.waves << "][" << in_rows_elems << "];\n";
    // Whole tiles of a 16-byte aligned x with a row stride of a multiple of
    // 8 elements go through LDS; others (the batch's last tile) load directly.
    o << "  bool const xvec = ((reinterpret_cast<uint64_t>(x) | uint64_t(ldx) * 2) & 15) == 0;\n";
    o << "  L.col0 = (int64_t(blockIdx.x) * " << NW << " + wave_id()) * " << WCOLS << ";\n";
    o << "  if (blockIdx.x < tiles && xvec && L.col0 + " << WCOLS << " <= batch) prefetch_rows_lds16<" << n_in0 << ", "
      << NT << ">(x, ldx, L, in_buf[wave_id()]);\n";
    // The LDS writes of these loads complete with vmcnt, which the compiler
    // does not track (fused_f16.h dma16): each tile's rows are waited for
    // explicitly, here for the first tile and before the output stores for
    // the next one (requested during the tile, so long landed).
    o << "  wait_vmem();\n";
  }
  o << "  for (int64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {\n";
  o << "    L.col0 = (tile * " << cfg.waves << " + wave_id()) * " << 16 * NT << ";\n";
  // Register-resident parameters may be hoisted out of the tile loop; otherwise
  // pin() hides the pointer's loop invariance so they are re-read per tile.
  o << "    " << F << " const* __restrict__ P = " << (cfg.params_in_registers ? "P0;\n" : "pin(P0);\n");
  int var = 0;
  auto fresh = [&]() { return "s" + std::to_string(var++); };
  std::string cur = fresh();
  int cur_n = p.layers.front().n_in;
  if (in_dma) {
    o << "    auto " << cur << " = xvec && L.col0 + " << WCOLS << " <= batch ? load_rows_lds16<" << cur_n << ", " << NT
      << ", E>(in_buf[wave_id()], L) : load_rows_h<" << cur_n << ", " << NT << ">(x, ldx, L);\n";
    o << "    wait_lds();\n";
    o << "    Lane Ln = L;\n    Ln.col0 = ((tile + gridDim.x) * " << NW << " + wave_id()) * " << WCOLS << ";\n";
    o << "    bool const pre_next = tile + gridDim.x < tiles && xvec && Ln.col0 + " << WCOLS << " <= batch;\n";
    if (hook_dense < 0) o << "    " << prefetch_next << "\n";
  } else if (half) o << "    auto " << cur << " = load_rows_h<" << cur_n << ", " << NT << ">(x, ldx, L);\n";
  else o << "    auto " << cur << " = " << (in_k.empty() ? "load_rows<" : "load_rows_k<") << cur_n << ">(x, ldx, L);\n";
  std::map<int, std::pair<std::string, int>> saved;  // slot -> (expression, width)
  // The logistic family runs on the hardware transcendentals (pointwise.h),
  // except in F64 plans, which keep the libm forms.
  auto act = [&](Step const& st) { return dbl ? act_expr(st, true) : act_fast_expr(st); };
  // fp32 view of the state for barrier ops: the state itself (fp32 path) or a
  // widened copy that is rounded back afterwards (16-bit path).
  auto open32 = [&]() -> std::string {
    if (!half) return cur;
    o << "    {\n    auto f = to_f32(" << cur << ");\n";
    return "f";
  };
  auto close32 = [&]() {
    if (half) o << "    " << cur << " = to_h<E>(f);\n    }\n";
  };
  auto epilogue = [&](std::string const& v, int n, int begin, int count) {
    bool pad = false;
    for (int s = 0; s < count; s++) {
      Step const& st = p.steps[begin + s];
      if (st.act == ACT_BIAS) {
        o << "    add_rows<" << tiles(n) << ">(" << v << ", " << vec(st.off, n) << ", L);\n";
      } else if (act_has_param(st.act)) {
        o << "    map_const<" << tiles(n) << ">(" << v << ", " << vec(st.off, n) << ", L, [](" << F << " v, " << F << " c) { return "
          << const_expr(st) << "; });\n";
        if (!zero_at_zero(st.act)) pad = true;
      } else {
        o << "    map<" << tiles(n) << ">(" << v << ", [](" << F << " v) { return " << act(st) << "; });\n";
        if (!zero_at_zero(st.act)) pad = true;
      }
    }
    if (pad && n % 16) o << "    zero_pad<" << n << ", " << tiles(n) << ">(" << v << ", L);\n";
  };
  std::string dense_hook;  // closes a dense_hs call that takes the prefetch hook
  bool pad_ok = true;      // false for a transposed tile
  for (Op const& op : p.ops) {
    o << "    // op code " << op.code << "\n";
    switch (op.code) {
      case OP_DENSE: {
        // Bias and activations run per output tile inside the contraction.
        std::string const nv = fresh();
        int const n = op.n_out;
        bool pad = false;
        // A generated Dense's bias seeds the fp32 accumulator (sum = bias first);
        // 16-bit plans seed any leading bias (their tolerance is that of the
        // 16-bit rounding, and the add then costs no VALU op).
        bool const lead_bias = op.epi_count > 0 && p.steps[op.epi_begin].act == ACT_BIAS;
        bool const seed = lead_bias && (half || (op.aux & DENSE_BIAS_FIRST));
        if (half) {
          bool const tr = out_transposed && &op == &p.ops.back();
          bool const hook = static_cast<int>(dense_index) == hook_dense;
          std::string const init = !seed ? "SeedZero{}"
                                   : tr  ? "SeedRowsT{" + vec(p.steps[op.epi_begin].off, n) + ", L.c}"
                                         : "SeedRows{" + vec(p.steps[op.epi_begin].off, n) + ", L.g}";
          dense_index++;
          o << "    auto " << nv << " = dense_hs<" << tiles(op.n_in) << ", " << tiles(n) << ", " << NT << ", "
            << cfg.waves << (tr || hook ? tr ? ", true" : ", false" : "") << (hook ? ", 0" : "") << ">(" << cur
            << ", st, L, " << init << ", [&](int mo, floatx4 (&t)[" << NT << "], Vec<E>::x4 (&o)[" << NT
            << "]) {\n";
          if (hook) dense_hook = "    }, [&] { " + prefetch_next + " });\n";
          if (tr) pad_ok = false;
        } else {
          std::string const init = seed ? "bias_rows<" + std::to_string(tiles(n)) + ">(" + vec(p.steps[op.epi_begin].off, n) + ", L)"
                                        : "zeros<" + std::to_string(tiles(n)) + ">()";
          o << "    auto " << nv << " = "
            << (epi_interleave > 0 ? "dense_ep_il<" + std::to_string(epi_interleave) + ", " : std::string("dense_ep<"))
            << tiles(op.n_in) << ", " << tiles(n) << k_steps(op.woff, op.n_in) << ">(" << cur << ", P + "
            << op.woff << ", " << init << ", L, [&](int mo, " << F4 << " (&t)[" << NT << "]) {\n";
        }
        for (int s = seed ? 1 : 0; s < op.epi_count; s++) {
          Step const& st = p.steps[op.epi_begin + s];
          if (st.act == ACT_BIAS) {
            o << "      tile_add_rows(t, " << vec(st.off, n) << ", mo, L);\n";
          } else if (act_has_param(st.act)) {
            o << "      tile_const(t, " << vec(st.off, n) << ", mo, L, [](" << F
              << " v, " << F << " c) { return " << const_expr(st) << "; });\n";
            if (!zero_at_zero(st.act)) pad = true;
          } else {
            o << "      tile_map(t, [](" << F << " v) { return " << act(st) << "; });\n";
            if (!zero_at_zero(st.act)) pad = true;
          }
        }
        // Padding rows of the output: zero weights times an infinite or NaN
        // input make them NaN, and a later contraction would read them
        // (zero weights times NaN), so they are zeroed unless nothing reads
        // them -- the plan's last op, whose store stops at row n, or a
        // transposed tile, whose padding rows are never read nor stored.
        if (n % 16 && pad_ok && &op != &p.ops.back()) pad = true;
        if (pad && n % 16 && pad_ok) o << "      if (mo == " << tiles(n) - 1 << ") tile_zero_pad<" << n << ">(t, mo, L);\n";
        if (half) o << "      tile_round<E>(t, o);\n";
        o << (dense_hook.empty() ? "    });\n" : dense_hook);
        dense_hook.clear();
        pad_ok = true;
        cur = nv;
        cur_n = n;
        break;
      }
      case OP_POINTWISE: {
        std::string const f = open32();
        epilogue(f, cur_n, op.epi_begin, op.epi_count);
        close32();
        break;
      }
      case OP_LAYER_NORM: {
        std::string const f = open32();
        o << "    layer_norm<" << cur_n << ", " << tiles(cur_n) << ">(" << f << ", " << vec(op.woff, cur_n) << ", "
          << vec(op.boff, cur_n) << ", " << lit(op.f0) << ", L);\n";
        close32();
        break;
      }
      case OP_SOFTMAX:
      case OP_LOG_SOFTMAX: {
        std::string const f = open32();
        o << "    softmax<" << cur_n << ", " << (op.code == OP_LOG_SOFTMAX ? "true" : "false") << ">(" << f << ", L);\n";
        if (cur_n % 16) o << "    zero_pad<" << cur_n << ", " << tiles(cur_n) << ">(" << f << ", L);\n";
        close32();
        break;
      }
      case OP_MIN_MAX: {
        std::string const f = open32();
        o << "    min_max<" << cur_n << ", " << tiles(cur_n) << ">(" << f << ", " << lit(op.f0) << ", "
          << lit(op.f1) << ", " << lit(op.f2) << ", L);\n";
        if (cur_n % 16) o << "    zero_pad<" << cur_n << ", " << tiles(cur_n) << ">(" << f << ", L);\n";
        close32();
        break;
      }
      case OP_SAVE: {
        if (cfg.saved_in_lds) {
          o << "    save_lds<" << tiles(cur_n) << ">(" << cur << ", SV + " << slot_off[op.slot] << ", L);\n";
          saved[op.slot] = {"load_lds<" + std::to_string(tiles(cur_n)) + ">(SV + " + std::to_string(slot_off[op.slot]) +
                                ", L)",
                            cur_n};
        } else {
          std::string const sv = "sv" + std::to_string(op.slot) + "_" + std::to_string(var++);
          o << "    auto " << sv << " = " << cur << ";\n";
          saved[op.slot] = {sv, cur_n};
        }
        break;
      }
      case OP_ADD:
        if (cfg.saved_in_lds) {
          o << "    add_lds<" << tiles(cur_n) << ">(" << cur << ", SV + " << slot_off[op.slot] << ", L);\n";
        } else if (half) {
          std::string const f = open32();
          o << "    add(" << f << ", to_f32(" << saved[op.slot].first << "));\n";
          close32();
        } else {
          o << "    add(" << cur << ", " << saved[op.slot].first << ");\n";
        }
        break;
      case OP_CONCAT: {
        auto const& sv = saved[op.slot];
        std::string const nv = fresh();
        // after: [state; saved], else [saved; state] (ponni_Binop_Concatenate.h:63-86)
        std::string const first = op.aux ? cur : sv.first, second = op.aux ? sv.first : cur;
        int const n1 = op.aux ? cur_n : sv.second, n2 = op.aux ? sv.second : cur_n;
        if (n1 % 16 == 0) {
          o << "    auto " << nv << " = " << (half ? "concat_h<" : "concat<") << tiles(n1) << ", " << tiles(n2)
            << ">(" << first << ", " << second << ");\n";
        } else if (half) {
          // (16-bit values are exact in fp32: the moves round nothing)
          o << "    auto " << nv << " = to_h<E>(concat_any<" << n1 << ", " << n2 << ">(to_f32(" << first
            << "), to_f32(" << second << "), L));\n";
        } else {
          o << "    auto " << nv << " = concat_any<" << n1 << ", " << n2 << ">(" << first << ", " << second
            << ", L);\n";
        }
        cur = nv;
        cur_n = op.n_out;
        break;
      }
      case OP_PROJ_ADD: {
        // proj = b + W^T saved (bias first, ponni_Binop_Projection_Add.h:91-92); out = in + proj.
        auto const& sv = saved[op.slot];
        if (half) {
          o << "    proj_add_h<" << tiles(sv.second) << ", " << tiles(cur_n) << ", " << cur_n << ">(" << cur << ", " << sv.first
            << ", reinterpret_cast<E const*>(P + " << op.woff << "), " << vec(op.boff, cur_n) << ", L);\n";
        } else {
          // The bias seeds the accumulators; each finished tile adds the
          // state's tile (proj + in, the same sum as in + proj).
          std::string const nv = fresh();
          o << "    auto " << nv << " = "
            << (epi_interleave > 0 ? "dense_ep_il<" + std::to_string(epi_interleave) + ", " : std::string("dense_ep<"))
            << tiles(sv.second) << ", " << tiles(cur_n) << k_steps(op.woff, sv.second) << ">(" << sv.first
            << ", P + " << op.woff << ", bias_rows<" << tiles(cur_n) << ">(" << vec(op.boff, cur_n)
            << ", L), L, [&](int mo, " << F4 << " (&t)[" << NT << "]) { tile_add_state(t, " << cur << ", mo);"
            << (cur_n % 16 ? " if (mo == " + std::to_string(tiles(cur_n) - 1) + ") tile_zero_pad<" +
                                 std::to_string(cur_n) + ">(t, mo, L);"
                           : std::string())
            << " });\n";
          cur = nv;
        }
        break;
      }
      case OP_LOAD: {
        auto const& sv = saved[op.slot];
        std::string const nv = fresh();
        o << "    auto " << nv << " = " << sv.first << ";\n";
        cur = nv;
        cur_n = sv.second;
        break;
      }
      case OP_BINARY: {
        // out = f(x, y), x the left operand; a one-feature operand broadcasts.
        auto const& sv = saved[op.slot];
        bool const saved_left = op.aux & BIN_SAVED_LEFT;
        bool const state_scalar = op.aux & BIN_STATE_SCALAR, saved_scalar = op.aux & BIN_SAVED_SCALAR;
        std::string const nv = fresh();
        std::string const a = half ? "to_f32(" + cur + ")" : cur;
        std::string const b = half ? "to_f32(" + sv.first + ")" : sv.first;
        std::string const lhs = saved_left ? b : a, rhs = saved_left ? a : b;
        bool const lhs_scalar = saved_left ? saved_scalar : state_scalar;
        bool const rhs_scalar = saved_left ? state_scalar : saved_scalar;
        std::string call = "binary<" + std::to_string(op.n_out) + ", " + (lhs_scalar ? "true" : "false") + ", " +
                           (rhs_scalar ? "true" : "false") + ">(" + lhs + ", " + rhs +
                           ", L, [](" + F + " x, " + F + " y) { return " + binary_expr(op.aux & 0xff) + "; })";
        if (half) call = "to_h<E>(" + call + ")";
        o << "    auto " << nv << " = " << call << ";\n";
        cur = nv;
        cur_n = op.n_out;
        break;
      }
      case OP_SELECT: {
        // cond != 0 ? a : b; a constant operand is its vector broadcast over
        // the tile's columns, a one-feature operand broadcasts over features.
        std::string arg[3];
        int consts = 0;
        for (int k = 0; k < 3; k++) {
          int const code = sel_src(op.aux, k);
          if (code == 3) {
            arg[k] = fresh();
            o << "    auto " << arg[k] << " = bias_rows<" << tiles(op.n_out) << ", " << NT << ">("
              << vec(consts++ == 0 ? op.woff : op.boff, op.n_out) << ", L);\n";
            continue;
          }
          std::string const& e =
              code == 0 ? cur : saved[code == 1 ? op.slot : static_cast<int>(op.f0)].first;
          arg[k] = half ? "to_f32(" + e + ")" : e;
        }
        auto flag = [&](int bit) { return (op.aux & bit) ? std::string("true") : std::string("false"); };
        std::string call = "select3<" + std::to_string(op.n_out) + ", " + flag(SEL_COND_SCALAR) + ", " +
                           flag(SEL_A_SCALAR) + ", " + flag(SEL_B_SCALAR) + ">(" + arg[0] + ", " + arg[1] + ", " +
                           arg[2] + ", L)";
        if (half) call = "to_h<E>(" + call + ")";
        std::string const nv = fresh();
        o << "    auto " << nv << " = " << call << ";\n";
        cur = nv;
        cur_n = op.n_out;
        break;
      }
      case OP_REDUCE: {
        std::string const nv = fresh();
        std::string call = "reduce<" + std::to_string(op.aux) + ", " + std::to_string(cur_n) + ", " +
                           (half ? "true" : "false") + ">(" +
                           (half ? "to_f32(" + cur + ")" : cur) + ", L)";
        if (half) call = "to_h<E>(" + call + ")";
        o << "    auto " << nv << " = " << call << ";\n";
        cur = nv;
        cur_n = 1;
        break;
      }
      default:
        break;
    }
  }
  // Before the output stores: the input rows requested for the next tile
  // have landed (with staging, every request but the last chunk's is done,
  // and the rows were requested before it).
  if (half && in_dma)
    o << (stage_bytes > 0 ? "    wait_vmem_n<chunk_requests<" + NW + ">()>();\n" : std::string("    wait_vmem();\n"));
  if (out_transposed) o << "    store_rows_ht<" << cur_n << ">(" << cur << ", y, ldy, L, yvec);\n";
  else if (half) o << "    store_rows_h<" << cur_n << ">(" << cur << ", y, ldy, L);\n";
  else o << "    store_rows<" << cur_n << ">(" << cur << ", y, ldy, L);\n";
  o << "  }\n}\n";
  if (!vec_lds.empty()) {
    head << "  __shared__ floatx4 lds_vec[" << vec_total / 4 << "];\n";
    for (auto const& kv : vec_lds)
      head << "  stage_vec(lds_vec + " << kv.second.first / 4 << ", gparams + " << kv.first << ", "
           << kv.second.second / 4 << ");\n";
    head << "  __syncthreads();\n";
    head << "  float const* __restrict__ VP = reinterpret_cast<float const*>(lds_vec);\n";
  }
  cfg.vec_bytes = vec_total * 4;
  cfg.lds_total = stage_bytes + (in_dma ? in_dma_bytes : 0) + cfg.vec_bytes + static_cast<int>(cfg.lds_bytes);
  return head.str() + o.str();
}
}  // namespace

// ---- generated NARROW kernels ---------------------------------------------
// A narrow chain (every width <= 16) as straight-line code over
// narrow_jit.h: one lane owns V consecutive samples, parameters in the NARROW
// packing at constant offsets, vector row loads and stores.
namespace {

int narrow_samples_per_lane(ponni_plan_s const& p) {
  bool const half = p.dtype == PONNI_F16 || p.dtype == PONNI_BF16;
  if (p.dtype == PONNI_F64 || p.width_class >= 16) return 2;
  if (p.width_class >= 8) return 4;
  return half ? 8 : 4;
}

std::string narrow_source(ponni_plan_s const& p, FusedConfig& cfg) {
  int const W = p.width_class;
  int const V = narrow_samples_per_lane(p);
  bool const dbl = p.dtype == PONNI_F64;
  std::string const S = p.dtype == PONNI_F16 ? "_Float16" : p.dtype == PONNI_BF16 ? "__bf16" : dbl ? "double" : "float";
  std::string const R = dbl ? "double" : "float";  // compute type
  auto lit = [&](double v) { return dbl ? dlit(v) : flit(static_cast<float>(v)); };
  // U groups of V samples per lane, 256 * V samples apart, so that all of a
  // lane's input rows are in flight before its first FMA.
  int const U = 1;
  cfg = FusedConfig{};
  cfg.waves = 4;
  cfg.waves_per_simd = 4;
  cfg.columns_per_block = 256 * V * U;
  std::string const WV = ", " + std::to_string(W) + ">";
  auto tv = [&](int n) { return "<" + std::to_string(V) + ", " + std::to_string(n) + WV; };
  auto finish = [&](int n) { return "    finish<S, " + std::to_string(V) + ", " + std::to_string(n) + WV; };
  std::ostringstream o;
  o << "// generated by libponni_hip for one plan (NARROW)\n#include \"narrow_jit.h\"\n";
  o << "using namespace ponni_hip;\nusing namespace ponni_hip::narrowj;\ntypedef " << S << " S;\ntypedef " << R
    << " real;\n";
  // The chain on one group of V samples.
  o << "__device__ inline void chain(real (&s)[" << W << "][" << V << "], real const* __restrict__ P) {\n";
  for (int sl = 0; sl < p.num_slots; sl++)
    o << "  real sv" << sl << "[" << W << "][" << V << "] = {};\n";
  int cur_n = p.layers.front().n_in;
  auto steps = [&](std::string const& a, int n, int begin, int count) {
    for (int k = 0; k < count; k++) {
      Step const& st = p.steps[begin + k];
      if (act_has_param(st.act))
        o << "    with_vec" << tv(n) << "(" << a << ", P + " << st.off << ", [](real v, real c) { return "
          << const_expr(st) << "; });\n";
      else
        o << "    map" << tv(n) << "(" << a << ", [](real v) { return " << (dbl ? act_expr(st, true) : act_fast_expr(st))
          << "; });\n";
    }
  };
  for (Op const& op : p.ops) {
    o << "  {  // op code " << op.code << "\n";
    switch (op.code) {
      case OP_DENSE: {
        // Pointwise layers keep the width: the Matvec is n_in -> n_out.  A
        // generated Dense's bias (its first step) seeds the sum.
        int const K = op.n_in, N = op.n_out;
        bool const seed = op.aux & DENSE_BIAS_FIRST;
        o << "    real a[" << W << "][" << V << "];\n";
        if (seed)
          o << "    dense_bias<" << V << ", " << K << ", " << N << WV << "(a, s, P + " << op.woff << ", P + "
            << p.steps[op.epi_begin].off << ");\n";
        else
          o << "    dense<" << V << ", " << K << ", " << N << WV << "(a, s, P + " << op.woff << ");\n";
        steps("a", N, op.epi_begin + (seed ? 1 : 0), op.epi_count - (seed ? 1 : 0));
        o << finish(op.n_out) << "(s, a);\n";
        break;
      }
      case OP_LOAD:
        o << "    copy<" << V << WV << "(s, sv" << op.slot << ");\n";
        o << finish(op.n_out) << "(s, s);\n";
        break;
      case OP_BINARY:
        o << "    binary<" << V << ", " << op.n_out << ", " << W << ", " << op.aux << ">(s, sv" << op.slot << ");\n";
        o << finish(op.n_out) << "(s, s);\n";
        break;
      case OP_SELECT: {
        auto sv = [&](int code, int slot) {
          for (int k = 0; k < 3; k++)
            if (sel_src(op.aux, k) == code) return "sv" + std::to_string(slot);
          return std::string("s");  // unused operand
        };
        o << "    select3<" << V << ", " << op.n_out << ", " << W << ", " << op.aux << ">(s, " << sv(1, op.slot) << ", "
          << sv(2, static_cast<int>(op.f0)) << ", P + " << op.woff << ", P + " << op.boff << ");\n";
        o << finish(op.n_out) << "(s, s);\n";
        break;
      }
      case OP_REDUCE:
        o << "    reduce<" << V << ", " << cur_n << ", " << W << ", " << op.aux << ", "
          << (p.dtype == PONNI_F16 || p.dtype == PONNI_BF16 ? "true" : "false") << ">(s);\n";
        o << finish(1) << "(s, s);\n";
        break;
      case OP_POINTWISE:
        steps("s", cur_n, op.epi_begin, op.epi_count);
        o << finish(op.n_out) << "(s, s);\n";
        break;
      case OP_LAYER_NORM:
        o << "    layer_norm" << tv(cur_n) << "(s, P + " << op.woff << ", P + " << op.boff << ", real(" << lit(op.f0)
          << "));\n";
        o << finish(op.n_out) << "(s, s);\n";
        break;
      case OP_SOFTMAX:
      case OP_LOG_SOFTMAX:
        o << "    softmax<" << V << ", " << cur_n << ", " << W << ", " << (op.code == OP_LOG_SOFTMAX ? "true" : "false")
          << ">(s);\n";
        o << finish(op.n_out) << "(s, s);\n";
        break;
      case OP_MIN_MAX:
        o << "    min_max" << tv(cur_n) << "(s, real(" << lit(op.f0) << "), real(" << lit(op.f1) << "), real(" << lit(op.f2)
          << "));\n";
        o << finish(op.n_out) << "(s, s);\n";
        break;
      case OP_SAVE:
        o << "    copy<" << V << WV << "(sv" << op.slot << ", s);\n";
        o << finish(op.n_out) << "(s, s);\n";
        break;
      case OP_ADD:
        o << "    for (int f = 0; f < " << W << "; f++) for (int v = 0; v < " << V << "; v++) s[f][v] += sv" << op.slot
          << "[f][v];\n";
        o << finish(op.n_out) << "(s, s);\n";
        break;
      case OP_CONCAT:
        if (op.aux)
          o << "    concat<" << V << ", " << op.n_in << ", " << op.n_out << WV << "(s, s, sv" << op.slot << ");\n";
        else
          o << "    concat<" << V << ", " << op.n_out - op.n_in << ", " << op.n_out << WV << "(s, sv" << op.slot
            << ", s);\n";
        o << finish(op.n_out) << "(s, s);\n";
        break;
      case OP_PROJ_ADD:
        o << "    proj_add<" << V << ", " << op.n_in << ", " << op.aux << WV << "(s, sv" << op.slot << ", P + " << op.woff
          << ", P + " << op.boff << ");\n";
        o << finish(op.n_out) << "(s, s);\n";
        break;
      default:
        break;
    }
    o << "  }\n";
    cur_n = op.n_out;
  }
  o << "}\n";
  o << "extern \"C\" __global__ __launch_bounds__(256) void " << fused_kernel_name(p)
    << "(real const* __restrict__ P, S const* __restrict__ x, int64_t ldx, S* __restrict__ y, int64_t ldy, "
       "int64_t batch) {\n";
  o << "  constexpr int U = " << U << ", V = " << V << ";\n";
  o << "  bool const aligned = vec_ok<S, V>(x, ldx) && vec_ok<S, V>(y, ldy);\n";
  // Workgroups wholly inside the batch (all but the last) with vector-aligned
  // views take a path with no per-lane predicate, so every load is issued
  // before the first wait.
  o << "  if (aligned && (int64_t(blockIdx.x) + 1) * (U * 256 * V) <= batch) {\n";
  o << "    real s[U][" << W << "][V];\n";
  o << "#pragma unroll\n    for (int u = 0; u < U; u++)\n      load<S, V, " << p.layers.front().n_in << WV
    << "(s[u], x, ldx, ((int64_t(blockIdx.x) * U + u) * 256 + threadIdx.x) * V, batch, true);\n";
  o << "#pragma unroll\n    for (int u = 0; u < U; u++) chain(s[u], P);\n";
  o << "#pragma unroll\n    for (int u = 0; u < U; u++)\n      store<S, V, " << p.layers.back().n_out << WV
    << "(s[u], y, ldy, ((int64_t(blockIdx.x) * U + u) * 256 + threadIdx.x) * V, batch, true);\n";
  o << "    return;\n  }\n";
  o << "  real s[U][" << W << "][V];\n";
  o << "  int64_t b0[U];\n";
  o << "#pragma unroll\n  for (int u = 0; u < U; u++) {\n";
  o << "    b0[u] = ((int64_t(blockIdx.x) * U + u) * 256 + threadIdx.x) * V;\n";
  o << "    if (b0[u] < batch) load<S, V, " << p.layers.front().n_in << WV
    << "(s[u], x, ldx, b0[u], batch, aligned && b0[u] + V <= batch);\n  }\n";
  o << "#pragma unroll\n  for (int u = 0; u < U; u++)\n    if (b0[u] < batch) chain(s[u], P);\n";
  o << "#pragma unroll\n  for (int u = 0; u < U; u++)\n    if (b0[u] < batch) store<S, V, " << p.layers.back().n_out
    << WV << "(s[u], y, ldy, b0[u], batch, aligned && b0[u] + V <= batch);\n}\n";
  return o.str();
}

}  // namespace

std::string narrow_source_of(ponni_plan_s const& p, FusedConfig& cfg) { return narrow_source(p, cfg); }

bool narrow_jit_supports(ponni_plan_s const& p) {
  if (p.path != PONNI_PATH_NARROW || p.width_class <= 0) return false;
  if (p.num_slots > kNarrowJitMaxSlots) return false;
  for (Op const& op : p.ops)
    if (op.code == OP_EXTERNAL) return false;
  return true;
}

namespace {

// The code generator behind hipRTC: the libamd_comgr the process has loaded,
// else the one beside the loaded hipRTC library, which hipRTC loads at its
// first compile.  hipRTC reports one version for different code generators:
// torch ships its own hipRTC and comgr (older than the system ROCm's), which
// a Python process that imported torch uses, while a C++ program uses the
// system's, and their kernels differ in rounding (one fuses the last FMA
// with the conversion to fp16, the other rounds twice).
std::string compiler_identity() {
  std::string path;
  dl_iterate_phdr(
      [](dl_phdr_info* info, size_t, void* out) -> int {
        if (info->dlpi_name == nullptr || std::strstr(info->dlpi_name, "libamd_comgr") == nullptr) return 0;
        *static_cast<std::string*>(out) = info->dlpi_name;
        return 1;
      },
      &path);
  char buf[PATH_MAX];
  if (path.empty()) {
    Dl_info di{};
    if (dladdr(reinterpret_cast<void*>(&hiprtcCompileProgram), &di) != 0 && di.dli_fname != nullptr &&
        realpath(di.dli_fname, buf) != nullptr) {
      std::string dir(buf);
      dir = dir.substr(0, dir.rfind('/'));
      path = dir + "/libamd_comgr.so.3";
    }
  }
  if (path.empty() || realpath(path.c_str(), buf) == nullptr) return "comgr unknown";
  std::string id = std::string("comgr ") + buf;
  struct stat sb;
  if (stat(buf, &sb) == 0) id += " " + std::to_string(sb.st_size) + " " + std::to_string(sb.st_mtime);
  return id;
}

// Source, options, embedded headers, the run-time compiler's version and
// code generator: a compiler change (whose code generation the kernels'
// numerics depend on) never picks up an object another one wrote.
std::string cache_key(std::string const& src, bool contract) {
  std::string opts;
  for (auto const* o : jit_options(contract)) opts += std::string(o) + " ";
  int major = 0, minor = 0;
  if (hiprtcVersion(&major, &minor) == HIPRTC_SUCCESS)
    opts += "hiprtc " + std::to_string(major) + "." + std::to_string(minor) + " ";
  opts += compiler_identity() + " ";
  std::string hdrs;
  for (int i = 0; i < kJitHeaderCount; i++) hdrs += kJitHeaderTexts[i];
  char buf[32];
  std::snprintf(buf, sizeof(buf), "%016llx", static_cast<unsigned long long>(fnv(src + opts + hdrs)));
  return buf;
}

std::mutex g_code_mutex;
std::map<std::string, std::vector<char>> g_code;  // key -> code object

}  // namespace

namespace {

// Register use of the kernel in a gfx950 code object, read from its AMDGPU
// metadata note (msgpack map entries ".vgpr_count", ".agpr_count",
// ".vgpr_spill_count"); -1 when absent.
int metadata_int(std::vector<char> const& code, char const* key) {
  std::string const k = key;
  std::string pattern(1, static_cast<char>(0xa0 | k.size()));
  pattern += k;
  std::string const blob(code.begin(), code.end());
  size_t const at = blob.find(pattern);
  if (at == std::string::npos || at + pattern.size() >= blob.size()) return -1;
  auto const* b = reinterpret_cast<unsigned char const*>(blob.data()) + at + pattern.size();
  size_t const left = blob.size() - at - pattern.size();
  if (b[0] < 0x80) return b[0];
  if (b[0] == 0xcc && left >= 2) return b[1];
  if (b[0] == 0xcd && left >= 3) return (b[1] << 8) | b[2];
  return -1;
}

int compile_cached(ponni_plan_s const& p, std::string& key, std::vector<char>& code, std::string& error);

}  // namespace

// Occupancy is settled by measurement: the kernel is compiled at the
// estimated waves per SIMD; with register spills it is recompiled for one
// wave fewer, and when it fits the next occupancy's register budget (512 /
// waves, a multiple of 8) without spills it moves up one.
int fused_compile(ponni_plan_s& p, std::string& key, std::vector<char>& code, std::string& error) {
  if (p.path == PONNI_PATH_FUSED && p.fused_wps == 0) {
    FusedConfig est;
    (void)fused_source(p, est);
    int wps = est.waves_per_simd;
    auto spills_regs = [&](int w, int& spills, int& regs) -> int {
      p.fused_wps = w;
      int const st = compile_cached(p, key, code, error);
      if (st != PONNI_OK) return st;
      spills = metadata_int(code, ".vgpr_spill_count");
      int const v = metadata_int(code, ".vgpr_count"), a = metadata_int(code, ".agpr_count");
      regs = (v < 0 ? 512 : v) + (a < 0 ? 0 : a);
      return static_cast<int>(PONNI_OK);
    };
    // 16-bit plans keep two waves per SIMD with spilled registers: one wave
    // per SIMD halves the columns each staged weight chunk serves.  With one
    // column tile per wave (wider than 256 features) that costs more than any
    // spilling measured (fp16 64x512x512x64, 20 registers spilled: 3.28
    // against 5.25 ms; 40 -> 512 residual chain with a LayerNorm, 109: 3.60
    // against 4.84 ms; the same at 1024 features, 691: 8.9 against 11.8 ms);
    // with two, up to 64 (that chain at 192 / 256 features, 44 / 47
    // spilled: 13-16 % faster; a 256-wide chain of three residual blocks,
    // 328: 20 % slower).
    bool const half = p.dtype == PONNI_F16 || p.dtype == PONNI_BF16;
    auto tolerated = [&](int w) { return half && w == 2 ? fused_nt(p) == 1 ? INT_MAX : 64 : 0; };
    int spills = 0, regs = 0;
    int st = spills_regs(wps, spills, regs);
    if (st != PONNI_OK) return st;
    while (spills > tolerated(wps) && wps > 1) {
      wps--;
      st = spills_regs(wps, spills, regs);
      if (st != PONNI_OK) return st;
    }
    auto budget = [](int w) { return (512 / w) / 8 * 8; };
    if (spills == 0 && wps < 4 && regs <= budget(wps + 1)) {
      int up_spills = 0, up_regs = 0;
      st = spills_regs(wps + 1, up_spills, up_regs);
      if (st != PONNI_OK) return st;
      if (up_spills == 0) wps = wps + 1;
    }
    p.fused_wps = wps;
  }
  return compile_cached(p, key, code, error);
}

namespace {

int compile_cached(ponni_plan_s const& p, std::string& key, std::vector<char>& code, std::string& error) {
  FusedConfig cfg;
  std::string const src = fused_source(p, cfg);
  key = cache_key(src, contract_on(p));
  std::lock_guard<std::mutex> lock(g_code_mutex);
  auto it = g_code.find(key);
  if (it != g_code.end()) {
    code = it->second;
    return PONNI_OK;
  }
  std::string const dir = cache_dir();
  std::string const path = dir.empty() ? "" : dir + "/" + key + ".co";
  code.clear();
  if (!path.empty()) {
    std::ifstream in(path, std::ios::binary);
    if (in) code.assign(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>());
  }
  if (code.empty()) {
    std::string log;
    if (!compile(src, contract_on(p), code, log)) {
      error = "hipRTC failed to compile the fused kernel:\n" + log;
      return PONNI_ERR_DEVICE;
    }
    if (!path.empty()) {
      ::mkdir(dir.c_str(), 0755);
      std::string const tmp = path + ".tmp" + std::to_string(::getpid());
      std::ofstream out(tmp, std::ios::binary);
      out.write(code.data(), static_cast<std::streamsize>(code.size()));
      out.close();
      if (out) std::rename(tmp.c_str(), path.c_str());
      else std::remove(tmp.c_str());
    }
  }
  g_code[key] = code;
  return PONNI_OK;
}

}  // namespace

int fused_prepare(ponni_plan_s& p, std::string& error) {
  std::string key;
  std::vector<char> code;
  int const st = fused_compile(p, key, code, error);
  if (st != PONNI_OK) return st;
  FusedConfig cfg;
  (void)fused_source(p, cfg);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    error = "no HIP device";
    return PONNI_ERR_DEVICE;
  }
  std::lock_guard<std::mutex> lock(g_mutex);
  auto it = g_modules.find({dev, key});
  if (it == g_modules.end()) {
    auto m = std::make_shared<Module>();
    hipError_t e = hipModuleLoadData(&m->module, code.data());
    if (e == hipSuccess) e = hipModuleGetFunction(&m->fn, m->module, fused_kernel_name(p).c_str());
    if (e == hipSuccess)
      e = hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&m->blocks_per_cu, m->fn, cfg.waves * 64, 0);
    if (e != hipSuccess) {
      error = std::string("loading the fused kernel failed: ") + hipGetErrorString(e);
      return PONNI_ERR_DEVICE;
    }
    it = g_modules.emplace(std::make_pair(dev, key), m).first;
  }
  p.fused_fn = it->second->fn;
  p.fused_blocks_per_cu = it->second->blocks_per_cu > 0 ? it->second->blocks_per_cu : 1;
  // The persistent grid's size, looked up once rather than at every launch.
  if (hipDeviceGetAttribute(&p.fused_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      p.fused_cus <= 0) {
    error = "no compute units";
    return PONNI_ERR_DEVICE;
  }
  p.fused_persistent = cfg.lds_bytes > 0 || cfg.vec_bytes > 0 || cfg.params_in_registers || cfg.persistent_loop;
  p.fused_columns_per_block = cfg.columns_per_block;
  p.fused_waves = cfg.waves;
  return PONNI_OK;
}

hipError_t fused_launch(ponni_plan_s const& p, LaunchArgs const& a, hipStream_t stream) {
  int64_t const blocks = (a.batch + p.fused_columns_per_block - 1) / p.fused_columns_per_block;
  int64_t grid = blocks;
  if (p.fused_persistent) {
    int64_t const resident = int64_t(p.fused_cus) * p.fused_blocks_per_cu;
    grid = blocks < resident ? blocks : resident;
  }
  void const* params = a.params;
  void const* x = a.x;
  void* y = a.y;
  int64_t ldx = a.ld_x, ldy = a.ld_y, batch = a.batch;
  void* args[] = {&params, &x, &ldx, &y, &ldy, &batch};
  unsigned const threads = 64u * unsigned(p.fused_waves);
  bool const timed = a.ev_start != nullptr || a.ev_stop != nullptr;
  // The extended launch takes the global work size in 32 bits; a grid
  // beyond that is timed by events recorded around an ordinary launch.
  if (timed && uint64_t(grid) * threads <= UINT32_MAX)
    return hipExtModuleLaunchKernel(p.fused_fn, static_cast<uint32_t>(uint64_t(grid) * threads), 1, 1, threads, 1, 1,
                                    0, stream, args, nullptr, a.ev_start, a.ev_stop, 0);
  if (timed && a.ev_start != nullptr) {
    hipError_t const e = hipEventRecord(a.ev_start, stream);
    if (e != hipSuccess) return e;
  }
  hipError_t const e =
      hipModuleLaunchKernel(p.fused_fn, static_cast<unsigned>(grid), 1, 1, threads, 1, 1, 0, stream, args, nullptr);
  if (e != hipSuccess || !timed || a.ev_stop == nullptr) return e;
  return hipEventRecord(a.ev_stop, stream);
}

}  // namespace ponni_hip
