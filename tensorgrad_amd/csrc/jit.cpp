// Generated fused-group kernels: source generation from a group program, and a
// process-wide hipRTC compile / module cache. See jit.h.
#include "jit.h"

#include <hip/hiprtc.h>

#include <cstdio>
#include <cstdlib>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <sstream>
#include <stdexcept>

namespace tgk {

namespace {

// fused_dev.h as text: the prelude of every hipRTC program.
const char* const kFusedDevSource =
#include "fused_dev_src.inc"
    ;
// gemm_dev.h as text: added to programs that hold GEMM kernels with fused epilogues.
const char* const kGemmDevSource =
#include "gemm_dev_src.inc"
    ;

std::string dlit(double v) {   // exact (hexadecimal) double literal
  char b[64];
  snprintf(b, sizeof b, "%a", v);
  return b;
}
std::string ulit(int64_t v) { return std::to_string(v) + "u"; }

bool binary_op(int op) {
  switch (op) {
    case FO_FADD: case FO_FSUB: case FO_FMUL: case FO_FDIV: case FO_RELU_GRAD:
    case FO_ADD: case FO_SUB: case FO_MUL: case FO_DIV: case FO_MIN: case FO_MAX: case FO_LESS: case FO_GREATER:
      return true;
    default:
      return false;
  }
}

uint64_t fnv1a(const std::string& s) {
  uint64_t h = 1469598103934665603ull;
  for (unsigned char c : s) { h ^= c; h *= 1099511628211ull; }
  return h;
}

// Linear offset of operand k over coordinates c0..c{rank-1}.
std::string offset_expr(const FusedProgram& p, int k) {
  std::string s;
  for (int d = 0; d < p.rank; ++d) {
    const int64_t st = p.in_strides[k][d];
    if (st == 0) continue;
    if (!s.empty()) s += " + ";
    s += "c" + std::to_string(d) + (st == 1 ? "" : " * " + ulit(st));
  }
  return s.empty() ? "0u" : s;
}

// Coordinates of `idx` over the iteration dims p.div[0..rank) (row-major).
void emit_coords(std::ostringstream& o, const FusedProgram& p, const char* idx, const char* ind) {
  o << ind << "unsigned c0";
  for (int d = 1; d < p.rank; ++d) o << ", c" << d;
  o << ";\n" << ind << "{\n" << ind << "  unsigned rem = " << idx << ";\n";
  for (int d = p.rank - 1; d >= 1; --d) {
    const std::string D = ulit(p.div[d].d);
    o << ind << "  c" << d << " = rem % " << D << "; rem /= " << D << ";\n";
  }
  o << ind << "  c0 = rem;\n" << ind << "}\n";
}

}  // namespace

JitKernel fused_kernel(const FusedProgram& p, const FusedInstr* code, int64_t n) {
  const bool row = p.row_d > 0;
  const int64_t D = p.row_d;
  // Row form: one wavefront per row; lane l owns chunks j = 0 .. J-1 of V consecutive
  // columns, (l + 64 j) V .. (l + 64 j) V + V - 1, so every chunk is one V-wide access and
  // a wavefront's accesses of a chunk cover 256 V contiguous bytes.
  int V = 1;
  if (row && D % 4 == 0 && D >= 256) V = 4;
  else if (row && D % 2 == 0 && D >= 128) V = 2;
  const int J = row ? (int)((D + 64 * V - 1) / (64 * V)) : 0;
  const int N = row ? J * V : p.vec;   // elements per thread
  const char* I = "      ";
  // chunk j is live in lanes below this bound (-1: in every lane)
  auto chunk_lanes = [&](int j) -> int64_t {
    return (int64_t)64 * (j + 1) * V <= D ? -1 : (D + V - 1) / V - (int64_t)64 * j;
  };
  auto live = [&](int e) -> std::string {   // row form: condition for element e (empty = always)
    if (!row) return "";
    const int64_t l = chunk_lanes(e / V);
    return l < 0 ? "" : "lane < " + ulit(l);
  };
  auto col = [&](int e) -> std::string {   // row form: column of element e
    const int64_t c0 = (int64_t)64 * (e / V) * V + e % V;
    return (V == 1 ? std::string("lane") : "lane * " + ulit(V)) + (c0 ? " + " + ulit(c0) : std::string());
  };
  const char* vt = V == 4 ? "tgk::u32x4" : "tgk::u32x2";
  bool dropout = false;
  for (int q = 0; q < p.n_instr; ++q) dropout |= code[q].op == FO_DROPOUT;

  std::ostringstream o;
  o << "extern \"C\" __global__ void __launch_bounds__(256) @NAME@(const tgk::JitArgs A) {\n";
  o << "  const unsigned seed = " << (dropout ? "A.seed ? (unsigned)*A.seed : 0u" : "0u") << ";\n";
  if (row) {
    o << "  const unsigned lane = threadIdx.x & 63u;\n";
    o << "  for (unsigned rb = blockIdx.x * 4u; rb < " << ulit(n) << "; rb += gridDim.x * 4u) {\n";
    o << "    const unsigned r = rb + (threadIdx.x >> 6);\n";
    o << "    if (r < " << ulit(n) << ") {\n";   // wavefront-uniform: no lane of a wave diverges
    emit_coords(o, p, "r", I);
  } else {
    o << "  for (unsigned t = blockIdx.x * 256u + threadIdx.x; t < " << ulit(n) << "; t += gridDim.x * 256u) {\n";
    o << "    {\n";
    if (p.any_strided) emit_coords(o, p, "t", I);
  }

  // operand loads (all issued before any arithmetic)
  for (int k = 0; k < p.n_in; ++k) {
    const std::string x = "x" + std::to_string(k);
    const int64_t inner = p.in_inner[k];
    o << I << "unsigned " << x << "[" << N << "];\n";
    o << I << "{\n" << I << "  const unsigned* s = (const unsigned*)A.in[" << k << "];\n";
    if (row) {
      o << I << "  const unsigned b = " << offset_expr(p, k) << ";\n";
      bool vec = V > 1 && inner == 1;
      for (int d = 0; d < p.rank; ++d) vec = vec && p.in_strides[k][d] % V == 0;
      if (inner == 0) {
        o << I << "  const unsigned w = s[b];\n";
        for (int e = 0; e < N; ++e) o << I << "  " << x << "[" << e << "] = w;\n";
      } else if (vec) {
        for (int j = 0; j < J; ++j) {
          const std::string c = live(j * V);
          o << I << "  {\n" << I << "    " << vt << " w = {};\n";
          o << I << "    " << (c.empty() ? "" : "if (" + c + ") ") << "w = *(const " << vt << "*)(s + b + " << col(j * V)
            << ");\n";
          for (int u = 0; u < V; ++u) o << I << "    " << x << "[" << j * V + u << "] = w[" << u << "];\n";
          o << I << "  }\n";
        }
      } else {
        const std::string is = inner == 1 ? "" : " * " + ulit(inner);
        for (int e = 0; e < N; ++e) {
          const std::string c = live(e);
          const std::string ld = "s[b + (" + col(e) + ")" + is + "]";
          o << I << "  " << x << "[" << e << "] = " << (c.empty() ? ld : c + " ? " + ld + " : 0u") << ";\n";
        }
      }
    } else {
      const int m = p.in_mode[k];
      if (m == FM_CONTIG && N == 4) {
        o << I << "  const tgk::u32x4 w = *(const tgk::u32x4*)(s + t * 4u);\n";
        for (int e = 0; e < 4; ++e) o << I << "  " << x << "[" << e << "] = w[" << e << "];\n";
      } else if (m == FM_CONTIG) {
        o << I << "  " << x << "[0] = s[t];\n";
      } else if (m == FM_SCALAR || m == FM_STRIDED_B || (m == FM_STRIDED && inner == 0)) {
        o << I << "  const unsigned w = s[" << (m == FM_SCALAR ? std::string("0u") : offset_expr(p, k)) << "];\n";
        for (int e = 0; e < N; ++e) o << I << "  " << x << "[" << e << "] = w;\n";
      } else if (m == FM_STRIDED_V) {
        o << I << "  const tgk::u32x4 w = *(const tgk::u32x4*)(s + " << offset_expr(p, k) << ");\n";
        for (int e = 0; e < 4; ++e) o << I << "  " << x << "[" << e << "] = w[" << e << "];\n";
      } else {
        o << I << "  const unsigned b = " << offset_expr(p, k) << ";\n";
        for (int e = 0; e < N; ++e)
          o << I << "  " << x << "[" << e << "] = s[b" << (e ? " + " + ulit(e * inner) : "") << "];\n";
      }
    }
    o << I << "}\n";
  }

  // program: one SSA array per instruction; reg[] maps registers to current arrays
  std::vector<std::string> reg(64);
  for (int k = 0; k < p.n_in; ++k) reg[k] = "x" + std::to_string(k);
  auto R = [&](int r) -> const std::string& {
    if (r < 0 || r >= (int)reg.size() || reg[r].empty()) throw std::runtime_error("jit: read of an unset register");
    return reg[r];
  };
  const std::string elem = row ? "r * " + ulit(D) + " + (lane + 64u * (unsigned)(e / " + std::to_string(V) + ")) * " +
                                     ulit(V) + " + (unsigned)(e % " + std::to_string(V) + ")"
                               : "t * " + ulit(N) + " + (unsigned)e";
  for (int q = 0; q < p.n_instr; ++q) {
    const FusedInstr& in = code[q];
    const std::string v = "v" + std::to_string(q);
    o << I << "unsigned " << v << "[" << N << "];\n";
    if (in.op == FO_ROWSUM || in.op == FO_SOFTMAX_CAUSAL || in.op == FO_LOG_SOFTMAX) {
      if (!row) throw std::runtime_error("jit: row opcode in an element group");
      const std::string& a = R(in.a);
      o << I << "{\n";
      if (in.op == FO_ROWSUM) {
        // f64, each lane's chunks in order, then a wavefront butterfly (the interpreter's order)
        o << I << "  double s = 0.0;\n";
        for (int e = 0; e < N; ++e) {
          const std::string c = live(e);
          o << I << "  " << (c.empty() ? "" : "if (" + c + ") ") << "s += (double)tgk::bitsf(" << a << "[" << e << "]);\n";
        }
        o << I << "  s = tgk::wave_allsum(s);\n";
        o << I << "  const unsigned w = tgk::fbits((float)(s / " << dlit(in.imm) << "));\n";
        for (int e = 0; e < N; ++e) o << I << "  " << v << "[" << e << "] = w;\n";
      } else {
        const bool causal = in.op == FO_SOFTMAX_CAUSAL;
        if (causal) o << I << "  const unsigned rq = r % " << ulit(D) << ";\n";
        o << I << "  bool in_row[" << N << "];\n";
        for (int e = 0; e < N; ++e) {
          std::string c = live(e);
          if (causal) c = (c.empty() ? "" : c + " && ") + "(" + col(e) + ") <= rq";
          o << I << "  in_row[" << e << "] = " << (c.empty() ? "true" : c) << ";\n";
        }
        o << I << "  float mx = tgk::bitsf(0xff800000u);\n";
        o << I << "#pragma unroll\n" << I << "  for (int e = 0; e < " << N << "; ++e)\n"
          << I << "    if (in_row[e]) mx = fmaxf(mx, tgk::bitsf(" << a << "[e]));\n";
        o << I << "  mx = tgk::wave_allmax(mx);\n";
        o << I << "  double ex[" << N << "];\n" << I << "  double s = 0.0;\n";
        o << I << "#pragma unroll\n" << I << "  for (int e = 0; e < " << N << "; ++e) {\n"
          << I << "    ex[e] = in_row[e] ? exp((double)tgk::bitsf(" << a << "[e]) - (double)mx) : 0.0;\n"
          << I << "    if (in_row[e]) s += ex[e];\n" << I << "  }\n";
        o << I << "  s = tgk::wave_allsum(s);\n";
        if (causal) {
          o << I << "#pragma unroll\n" << I << "  for (int e = 0; e < " << N << "; ++e) " << v
            << "[e] = in_row[e] ? tgk::fbits((float)(ex[e] / s)) : 0u;\n";
        } else {
          o << I << "  const double ls = log(s) + (double)mx;\n";
          o << I << "#pragma unroll\n" << I << "  for (int e = 0; e < " << N << "; ++e) " << v
            << "[e] = tgk::fbits((float)((double)tgk::bitsf(" << a << "[e]) - ls));\n";
        }
      }
      o << I << "}\n";
    } else if (in.op == FO_ONEHOT) {
      if (!row) throw std::runtime_error("jit: row opcode in an element group");
      const char* one = in.dt == DT_I32 ? "1u" : "0x3f800000u";
      for (int e = 0; e < N; ++e)
        o << I << v << "[" << e << "] = (int)" << R(in.a) << "[" << e << "] == (int)(" << col(e) << ") ? " << one
          << " : 0u;\n";
    } else if (in.op == FO_WHERE) {
      o << I << "#pragma unroll\n" << I << "for (int e = 0; e < " << N << "; ++e) " << v << "[e] = " << R(in.a)
        << "[e] != 0u ? " << R(in.b) << "[e] : " << R(in.c) << "[e];\n";
    } else {
      const std::string b = binary_op(in.op) ? R(in.b) + "[e]" : std::string("0u");
      o << I << "#pragma unroll\n" << I << "for (int e = 0; e < " << N << "; ++e) " << v << "[e] = tgk::op_eval("
        << in.op << ", " << R(in.a) << "[e], " << b << ", " << in.ta << ", " << in.tb << ", " << in.dt << ", "
        << dlit(in.imm) << ", " << dlit(in.imm2) << ", " << in.salt << "u, seed, "
        << (in.op == FO_DROPOUT ? elem : std::string("0u")) << ");\n";
    }
    if (in.dst < 0 || in.dst >= (int)reg.size()) throw std::runtime_error("jit: register out of range");
    reg[in.dst] = v;
  }

  // stores
  for (int k = 0; k < p.n_out; ++k) {
    const std::string& v = R(p.out_reg[k]);
    o << I << "{\n" << I << "  unsigned* d = (unsigned*)A.out[" << k << "];\n";
    if (row && p.out_row[k]) {
      o << I << "  if (lane == 0u) d[r] = " << v << "[0];\n";
    } else if (row) {
      o << I << "  const unsigned b = r * " << ulit(D) << ";\n";
      if (V > 1) {
        for (int j = 0; j < J; ++j) {
          const std::string c = live(j * V);
          o << I << "  " << (c.empty() ? "" : "if (" + c + ") ") << "*(" << vt << "*)(d + b + " << col(j * V) << ") = ("
            << vt << "){";
          for (int u = 0; u < V; ++u) o << (u ? ", " : "") << v << "[" << j * V + u << "]";
          o << "};\n";
        }
      } else {
        for (int e = 0; e < N; ++e) {
          const std::string c = live(e);
          o << I << "  " << (c.empty() ? "" : "if (" + c + ") ") << "d[b + " << col(e) << "] = " << v << "[" << e
            << "];\n";
        }
      }
    } else if (N == 4) {
      o << I << "  *(tgk::u32x4*)(d + t * 4u) = (tgk::u32x4){" << v << "[0], " << v << "[1], " << v << "[2], " << v
        << "[3]};\n";
    } else {
      o << I << "  d[t] = " << v << "[0];\n";
    }
    o << I << "}\n";
  }
  o << "    }\n  }\n}\n";

  JitKernel k;
  std::string body = o.str();
  char nm[32];
  snprintf(nm, sizeof nm, "tg_%016llx", (unsigned long long)fnv1a(body));
  k.name = nm;
  k.body = body.replace(body.find("@NAME@"), 6, k.name);
  const int64_t blocks = row ? (n + 3) / 4 : (n + 255) / 256;
  k.grid = blocks < 16384 ? blocks : 16384;
  return k;
}

JitKernel gemm_epi_kernel(const FusedProgram& p, const FusedInstr* code, const GemmEpiCfg& c) {
  if (p.row_d > 0 || p.vec != 1) throw std::runtime_error("jit: GEMM epilogue needs an element program of one element");
  bool dropout = false;
  for (int q = 0; q < p.n_instr; ++q) dropout |= code[q].op == FO_DROPOUT;
  const char* I = "    ";
  std::ostringstream o;
  // The epilogue functor: element (gm, gn) of the product is element t = gm * N + gn of
  // the group's iteration space (the product is contiguous and read in that order).
  // Two phases (gemm_tile's kPrefetch): load() reads the group's other inputs for an
  // element, operator() computes from them and the accumulator value and stores.
  o << "namespace {\nstruct @NAME@_epi {\n  tgk::JitArgs A;\n  unsigned seed;\n";
  o << "  static constexpr bool kPrefetch = true;\n";
  // kColSum: operator() returns output colsum_out's value, whose column sums gemm_tile totals
  if (c.colsum_out >= p.n_out) throw std::runtime_error("jit: column-sum output out of range");
  o << "  static constexpr bool kColSum = " << (c.colsum_out >= 0 ? "true" : "false") << ";\n";
  o << "  struct Pre { unsigned x[" << std::max(1, p.n_in) << "]; };\n";
  o << "  __device__ __forceinline__ Pre load(const tgk::GemmDesc&, int64_t gm, int64_t gn) const {\n";
  o << I << "Pre q;\n";
  o << I << "const unsigned t = (unsigned)gm * " << ulit(c.N) << " + (unsigned)gn;\n";
  if (p.any_strided) emit_coords(o, p, "t", I);
  for (int k = 0; k < p.n_in; ++k) {
    if (k == c.h_in) continue;
    const int m = p.in_mode[k];
    o << I << "q.x[" << k << "] = ((const unsigned*)A.in[" << k << "])[";
    if (m == FM_CONTIG) o << "t";
    else if (m == FM_SCALAR) o << "0u";
    else o << offset_expr(p, k);
    o << "];\n";
  }
  o << I << "(void)t;\n" << I << "return q;\n  }\n";
  o << "  __device__ __forceinline__ float operator()(const tgk::GemmDesc& d, int64_t, int64_t, int64_t gm, int64_t gn, "
       "float value, const Pre& q) const {\n";
  if (c.store_c) o << I << "d.C[gm * d.sCm + gn * d.sCn] = value;\n";
  o << I << "const unsigned t = (unsigned)gm * " << ulit(c.N) << " + (unsigned)gn;\n";
  o << I << "(void)t;\n";
  for (int k = 0; k < p.n_in; ++k) {
    const std::string x = "x" + std::to_string(k);
    if (k == c.h_in) o << I << "const unsigned " << x << " = tgk::fbits(value);\n";
    else o << I << "const unsigned " << x << " = q.x[" << k << "];\n";
  }
  std::vector<std::string> reg(64);
  for (int k = 0; k < p.n_in; ++k) reg[k] = "x" + std::to_string(k);
  auto R = [&](int r) -> const std::string& {
    if (r < 0 || r >= (int)reg.size() || reg[r].empty()) throw std::runtime_error("jit: read of an unset register");
    return reg[r];
  };
  for (int q = 0; q < p.n_instr; ++q) {
    const FusedInstr& in = code[q];
    const std::string v = "v" + std::to_string(q);
    if (in.op == FO_ROWSUM || in.op == FO_SOFTMAX_CAUSAL || in.op == FO_LOG_SOFTMAX || in.op == FO_ONEHOT)
      throw std::runtime_error("jit: row opcode in a GEMM epilogue");
    if (in.op == FO_WHERE) {
      o << I << "const unsigned " << v << " = " << R(in.a) << " != 0u ? " << R(in.b) << " : " << R(in.c) << ";\n";
    } else {
      const std::string b = binary_op(in.op) ? R(in.b) : std::string("0u");
      o << I << "const unsigned " << v << " = tgk::op_eval(" << in.op << ", " << R(in.a) << ", " << b << ", " << in.ta
        << ", " << in.tb << ", " << in.dt << ", " << dlit(in.imm) << ", " << dlit(in.imm2) << ", " << in.salt
        << "u, seed, " << (in.op == FO_DROPOUT ? "t" : "0u") << ");\n";
    }
    if (in.dst < 0 || in.dst >= (int)reg.size()) throw std::runtime_error("jit: register out of range");
    reg[in.dst] = v;
  }
  for (int k = 0; k < p.n_out; ++k) o << I << "((unsigned*)A.out[" << k << "])[t] = " << R(p.out_reg[k]) << ";\n";
  if (c.colsum_out >= 0) o << I << "return tgk::bitsf(" << R(p.out_reg[c.colsum_out]) << ");\n";
  else o << I << "return 0.0f;\n";
  o << "  }\n};\n}  // namespace\n";
  o << "extern \"C\" __global__ void __launch_bounds__(" << c.nt
    << ") @NAME@(const tgk::gd::GemmArgs g, const tgk::JitArgs A) {\n";
  o << "  const @NAME@_epi e{A, " << (dropout ? "A.seed ? (unsigned)*A.seed : 0u" : "0u") << "};\n";
  if (c.skinny) {
    if (c.colsum_out >= 0) throw std::runtime_error("jit: no column partials in the skinny kernel");
    o << "  tgk::gd::skinny_tile<" << c.bm << ", " << (c.bk ? "true" : "false") << ">(g, e);\n}\n";
  } else if (c.tiny) {
    if (c.colsum_out >= 0) throw std::runtime_error("jit: no column partials in the tiny kernel");
    o << "  tgk::gd::tiny_tile<" << c.bm << ">(g, e);\n}\n";
  } else if (c.smallk) {
    o << "  tgk::gd::smallk_tile<" << c.bm << ", " << c.bk << ">(g, e);\n}\n";
  } else {
    o << "  tgk::gd::gemm_tile<" << c.bm << ", " << c.bn << ", " << c.bk << ", " << c.ns << ", "
      << (c.ak ? "true" : "false") << ", " << (c.bkf ? "true" : "false") << ", " << c.nt << ", " << c.kg;
    // a concatenation along k: the second A source and the partial last stage (KT, CAT);
    // the element-wise tile: both operands one element per lane (BDW, ADW) and KT
    if (c.cat) o << ", @NAME@_epi, false, false, true, false, true";
    else if (c.gen) o << ", @NAME@_epi, true, true, true";
    o << ">(g, tgk::gd::xcd_order(blockIdx.x, gridDim.x), e);\n}\n";
  }
  JitKernel k;
  std::string body = o.str();
  char nm[32];
  snprintf(nm, sizeof nm, "tg_g%016llx", (unsigned long long)fnv1a(body));
  k.name = nm;
  for (size_t pos; (pos = body.find("@NAME@")) != std::string::npos;) body.replace(pos, 6, k.name);
  k.body = body;
  k.grid = 0;   // set by the caller (the GEMM's tile count)
  k.gemm = true;
  return k;
}

namespace {

struct Cache {
  std::mutex mu;
  std::map<std::string, std::shared_ptr<std::vector<char>>> code_of;   // name -> code object holding it
  std::map<std::pair<int, const std::vector<char>*>, hipModule_t> modules;
  std::map<std::pair<int, std::string>, hipFunction_t> fns;
};
Cache& cache() {
  static Cache* c = new Cache();   // never destroyed: modules live until the process ends
  return *c;
}

std::shared_ptr<std::vector<char>> compile_program(const std::string& src) {
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), "tg_fused.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
    throw std::runtime_error("hipRTC: cannot create program");
  const char* opts[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  const hiprtcResult rc = hiprtcCompileProgram(prog, (int)(sizeof opts / sizeof opts[0]), opts);
  if (rc != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n, '\0');
    if (n) hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    throw std::runtime_error(std::string("hipRTC compile failed: ") + hiprtcGetErrorString(rc) + "\n" + log.substr(0, 4000));
  }
  size_t n = 0;
  hiprtcGetCodeSize(prog, &n);
  auto code = std::make_shared<std::vector<char>>(n);
  hiprtcGetCode(prog, code->data());
  hiprtcDestroyProgram(&prog);
  return code;
}

}  // namespace

void jit_compile(const std::vector<JitKernel>& ks, bool load) {
  Cache& c = cache();
  std::lock_guard<std::mutex> lock(c.mu);
  std::string src = kFusedDevSource;
  std::vector<std::string> fresh;
  std::set<std::string> seen;
  bool gemm = false;
  for (const auto& k : ks) {
    if (c.code_of.count(k.name) || !seen.insert(k.name).second) continue;
    fresh.push_back(k.name);
    gemm |= k.gemm;
  }
  if (gemm) src += std::string("\n") + kGemmDevSource;
  seen.clear();
  for (const auto& k : ks) {
    if (c.code_of.count(k.name) || !seen.insert(k.name).second) continue;
    src += "\n" + k.body;
  }
  if (!fresh.empty()) {
    // TG_JIT_DUMP=<file>: append each compiled program's source (for inspection).
    if (const char* path = std::getenv("TG_JIT_DUMP")) {
      if (FILE* f = fopen(path, "a")) {
        fputs(src.c_str(), f);
        fclose(f);
      }
    }
    auto code = compile_program(src);
    for (const auto& nm : fresh) c.code_of[nm] = code;
  }
  if (!load) return;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) throw std::runtime_error("jit: no current HIP device");
  for (const auto& k : ks) {
    const auto key = std::make_pair(dev, k.name);
    if (c.fns.count(key)) continue;
    const std::vector<char>* code = c.code_of.at(k.name).get();
    auto mk = std::make_pair(dev, code);
    auto it = c.modules.find(mk);
    if (it == c.modules.end()) {
      hipModule_t m;
      const hipError_t e = hipModuleLoadData(&m, code->data());
      if (e != hipSuccess) throw std::runtime_error(std::string("hipModuleLoadData: ") + hipGetErrorString(e));
      it = c.modules.emplace(mk, m).first;
    }
    hipFunction_t f;
    const hipError_t e = hipModuleGetFunction(&f, it->second, k.name.c_str());
    if (e != hipSuccess) throw std::runtime_error("hipModuleGetFunction(" + k.name + "): " + hipGetErrorString(e));
    c.fns[key] = f;
  }
}

hipFunction_t jit_function(const std::string& name) {
  Cache& c = cache();
  std::lock_guard<std::mutex> lock(c.mu);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) throw std::runtime_error("jit: no current HIP device");
  auto it = c.fns.find(std::make_pair(dev, name));
  if (it == c.fns.end()) throw std::runtime_error("jit: kernel " + name + " is not loaded");
  return it->second;
}

}  // namespace tgk
