// Fused element-wise groups for gfx950: one launch evaluates a chain of same-shape
// pointwise IR ops per output element, keeping intermediates in registers instead of
// one HBM round trip per op.
//
// Each group is a short straight-line program over f64 registers. Every register holds
// exactly the value the unfused op would have stored (f32-rounded, or an i32 / bool),
// so a fused group is bit-identical to running its ops one by one. Operands are loaded
// once per element through per-operand strides (0 on broadcast axes); results that are
// consumed outside the group are stored. The instruction stream is uniform across a
// wavefront, so the dispatch costs scalar work only; the kernel stays HBM-bound.
// Built with -ffp-contract=off.
#include "kernels.h"

#include <cmath>

namespace tgk {
namespace {

// General forms: one element through op_eval, kept out of line so the interpreter's body
// stays small.
__device__ __noinline__ uint32_t general_op(const FusedInstr in, uint32_t x, uint32_t y, uint32_t seed,
                                            uint32_t elem) {
  return op_eval(in.op, x, y, in.ta, in.tb, in.dt, in.imm, in.imm2, in.salt, seed, elem);
}

typedef const __attribute__((address_space(4))) FusedInstr* ConstCode;

// Register k of a thread is N consecutive LDS words at my + k * 256 * N, where
// my = regs + threadIdx.x * N: one 32/64/128-bit LDS access per register and thread,
// conflict-free across a wavefront, whatever the (wave-uniform) register index.
template <int N>
__device__ __forceinline__ void rload(const uint32_t* p, uint32_t (&v)[N]) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const u32x4 t = *reinterpret_cast<const u32x4*>(p + 4 * i);
      v[4 * i] = t[0]; v[4 * i + 1] = t[1]; v[4 * i + 2] = t[2]; v[4 * i + 3] = t[3];
    }
  } else if constexpr (N == 2) {
    const u32x2 t = *reinterpret_cast<const u32x2*>(p);
    v[0] = t[0]; v[1] = t[1];
  } else {
    v[0] = p[0];
  }
}
template <int N>
__device__ __forceinline__ void rstore(uint32_t* p, const uint32_t (&v)[N]) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      u32x4 t;
      t[0] = v[4 * i]; t[1] = v[4 * i + 1]; t[2] = v[4 * i + 2]; t[3] = v[4 * i + 3];
      *reinterpret_cast<u32x4*>(p + 4 * i) = t;
    }
  } else if constexpr (N == 2) {
    u32x2 t;
    t[0] = v[0]; t[1] = v[1];
    *reinterpret_cast<u32x2*>(p) = t;
  } else {
    p[0] = v[0];
  }
}

// The program interpreter shared by both kernel forms. A thread owns N elements. Element
// e has flat index elem0 + e * estride (the dropout hash index). Row form (TPR > 0): the
// TPR threads of a row hold its elements j = lane + e * TPR, bit e of `live` marks
// j < D of a real row, and FO_ROWSUM reduces a register over the row (f64, fixed order:
// each thread's elements in order, a wavefront butterfly, then the row's wavefronts in
// order through `part`).
template <int N, int TPR>
__device__ __forceinline__ void run_program(ConstCode code, int n_instr, uint32_t* my, uint32_t seed, uint32_t elem0,
                                            uint32_t estride, uint32_t live, double* part, uint32_t row_q = 0) {
#define R(k) (my + (k) * (256 * N))
#define TG_UN(EXPR)                                                \
  {                                                                \
    uint32_t X_[N], Z_[N];                                         \
    rload<N>(R(a), X_);                                            \
    _Pragma("unroll") for (int e = 0; e < N; ++e) {                \
      const uint32_t X = X_[e];                                    \
      Z_[e] = (EXPR);                                              \
    }                                                              \
    rstore<N>(R(dst), Z_);                                         \
    break;                                                         \
  }
#define TG_BIN(EXPR)                                               \
  {                                                                \
    uint32_t X_[N], Y_[N], Z_[N];                                  \
    rload<N>(R(a), X_);                                            \
    rload<N>(R(b), Y_);                                            \
    _Pragma("unroll") for (int e = 0; e < N; ++e) {                \
      const uint32_t X = X_[e], Y = Y_[e];                         \
      Z_[e] = (EXPR);                                              \
    }                                                              \
    rstore<N>(R(dst), Z_);                                         \
    break;                                                         \
  }
  for (int q = 0; q < n_instr; ++q) {
    const int op = code[q].op, a = code[q].a, b = code[q].b, dst = code[q].dst;
    switch (op) {
      // Inexpensive and frequent opcodes inline (constant opcode), the rest out of line.
      case FO_FADD: TG_BIN(op_eval(FO_FADD, X, Y, DT_F32, DT_F32, DT_F32, 0.0, 0.0, 0u, 0u, 0u))
      case FO_FSUB: TG_BIN(op_eval(FO_FSUB, X, Y, DT_F32, DT_F32, DT_F32, 0.0, 0.0, 0u, 0u, 0u))
      case FO_FMUL: TG_BIN(op_eval(FO_FMUL, X, Y, DT_F32, DT_F32, DT_F32, 0.0, 0.0, 0u, 0u, 0u))
      case FO_FDIV: TG_BIN(op_eval(FO_FDIV, X, Y, DT_F32, DT_F32, DT_F32, 0.0, 0.0, 0u, 0u, 0u))
      case FO_MULS: {
        const double s = code[q].imm;
        const int ta = code[q].ta;
        TG_UN(op_eval(FO_MULS, X, 0u, ta, DT_F32, DT_F32, s, 0.0, 0u, 0u, 0u))
      }
      case FO_ADDS: {
        const double s = code[q].imm;
        const int ta = code[q].ta;
        TG_UN(op_eval(FO_ADDS, X, 0u, ta, DT_F32, DT_F32, s, 0.0, 0u, 0u, 0u))
      }
      case FO_SQRT: TG_UN(op_eval(FO_SQRT, X, 0u, DT_F32, DT_F32, DT_F32, 0.0, 0.0, 0u, 0u, 0u))
      case FO_NEG: TG_UN(op_eval(FO_NEG, X, 0u, DT_F32, DT_F32, DT_F32, 0.0, 0.0, 0u, 0u, 0u))
      case FO_ABS: TG_UN(op_eval(FO_ABS, X, 0u, DT_F32, DT_F32, DT_F32, 0.0, 0.0, 0u, 0u, 0u))
      case FO_RELU: TG_UN(op_eval(FO_RELU, X, 0u, DT_F32, DT_F32, DT_F32, 0.0, 0.0, 0u, 0u, 0u))
      case FO_RELU_GRAD: TG_BIN(op_eval(FO_RELU_GRAD, X, Y, DT_F32, DT_F32, DT_F32, 0.0, 0.0, 0u, 0u, 0u))
      case FO_WHERE: {
        uint32_t C_[N], A_[N], B_[N];
        rload<N>(R(a), C_);
        rload<N>(R(b), A_);
        rload<N>(R(code[q].c), B_);
#pragma unroll
        for (int e = 0; e < N; ++e) A_[e] = C_[e] != 0u ? A_[e] : B_[e];
        rstore<N>(R(dst), A_);
        break;
      }
      case FO_COPY: TG_UN(op_eval(FO_COPY, X, 0u, DT_F32, DT_F32, DT_F32, 0.0, 0.0, 0u, 0u, 0u))
      // Frequent f64 transcendentals and dropout inline.
      case FO_EXP: TG_UN(op_eval(FO_EXP, X, 0u, DT_F32, DT_F32, DT_F32, 0.0, 0.0, 0u, 0u, 0u))
      case FO_LOG: TG_UN(op_eval(FO_LOG, X, 0u, DT_F32, DT_F32, DT_F32, 0.0, 0.0, 0u, 0u, 0u))
      case FO_TANH: TG_UN(op_eval(FO_TANH, X, 0u, DT_F32, DT_F32, DT_F32, 0.0, 0.0, 0u, 0u, 0u))
      case FO_ERF: TG_UN(op_eval(FO_ERF, X, 0u, DT_F32, DT_F32, DT_F32, 0.0, 0.0, 0u, 0u, 0u))
      case FO_DROPOUT: {
        const uint32_t salt = code[q].salt;
        const double pr = code[q].imm, sc = code[q].imm2;
        uint32_t X_[N];
        rload<N>(R(a), X_);
#pragma unroll
        for (int e = 0; e < N; ++e) X_[e] = dropout_bits(X_[e], seed, salt, pr, sc, elem0 + e * estride);
        rstore<N>(R(dst), X_);
        break;
      }
      case FO_ROWSUM: {
        if (TPR > 0) {
          uint32_t X_[N];
          rload<N>(R(a), X_);
          double s = 0.0;
#pragma unroll
          for (int e = 0; e < N; ++e)
            if ((live >> e) & 1u) s += (double)bitsf(X_[e]);
          s = wave_allsum(s);
          if (TPR > 64) {
            if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
            __syncthreads();
            const int w0 = (threadIdx.x / (TPR > 0 ? TPR : 1)) * (TPR / 64);
            double tsum = 0.0;
#pragma unroll
            for (int w = 0; w < TPR / 64; ++w) tsum += part[w0 + w];
            s = tsum;
            __syncthreads();
          }
          const uint32_t v = fbits((float)(s / code[q].imm));
#pragma unroll
          for (int e = 0; e < N; ++e) X_[e] = v;
          rstore<N>(R(dst), X_);
        }
        break;
      }
      case FO_ONEHOT: {
        if (TPR > 0) {
          const uint32_t one = code[q].dt == DT_I32 ? 1u : 0x3f800000u;
          const int32_t col0 = (int32_t)(threadIdx.x % TPR);
          TG_UN((int32_t)X == col0 + e * TPR ? one : 0u)
        }
        break;
      }
      // Row softmaxes, one wavefront per row (TPR == 64): the same arithmetic and
      // combination order as the standalone k_softmax_causal / k_log_softmax kernels.
      case FO_SOFTMAX_CAUSAL:
      case FO_LOG_SOFTMAX: {
        if (TPR == 64) {
          const bool causal = op == FO_SOFTMAX_CAUSAL;
          uint32_t X_[N];
          rload<N>(R(a), X_);
          const uint32_t lane = threadIdx.x & 63;
          bool in_row[N];
          float mx = -INFINITY;
#pragma unroll
          for (int e = 0; e < N; ++e) {
            in_row[e] = ((live >> e) & 1u) && (!causal || lane + e * 64 <= row_q);
            if (in_row[e]) mx = fmaxf(mx, bitsf(X_[e]));
          }
          mx = wave_allmax(mx);
          double ex[N];
          double s = 0.0;
#pragma unroll
          for (int e = 0; e < N; ++e) {
            ex[e] = in_row[e] ? exp((double)bitsf(X_[e]) - (double)mx) : 0.0;
            if (in_row[e]) s += ex[e];
          }
          s = wave_allsum(s);
          if (causal) {
#pragma unroll
            for (int e = 0; e < N; ++e) X_[e] = in_row[e] ? fbits((float)(ex[e] / s)) : 0u;
          } else {
            const double ls = log(s) + (double)mx;
#pragma unroll
            for (int e = 0; e < N; ++e) X_[e] = fbits((float)((double)bitsf(X_[e]) - ls));
          }
          rstore<N>(R(dst), X_);
        }
        break;
      }
      default: {
        FusedInstr in;
        in.op = op; in.dst = dst; in.a = a; in.b = b; in.c = code[q].c;
        in.dt = code[q].dt; in.ta = code[q].ta; in.tb = code[q].tb; in.salt = code[q].salt;
        in.imm = code[q].imm; in.imm2 = code[q].imm2;
        uint32_t X_[N], Y_[N];
        rload<N>(R(a), X_);
        rload<N>(R(b), Y_);
#pragma unroll
        for (int e = 0; e < N; ++e) X_[e] = general_op(in, X_[e], Y_[e], seed, elem0 + e * estride);
        rstore<N>(R(dst), X_);
        break;
      }
    }
  }
#undef TG_UN
#undef TG_BIN
#undef R
}

// Element form: thread t evaluates elements VEC*t .. VEC*t + VEC - 1 of the (row-major)
// iteration space.
template <int VEC>
__global__ __launch_bounds__(256) void k_fused(const FusedProgram p, uint32_t nv) {
  extern __shared__ __attribute__((aligned(16))) uint32_t regs[];   // nregs * VEC * 256 words
  uint32_t* const my = regs + threadIdx.x * VEC;
  const uint32_t seed = p.seed ? (uint32_t)*p.seed : 0u;
  const ConstCode code = (ConstCode)(uintptr_t)p.code;
  for (uint32_t t = blockIdx.x * 256u + threadIdx.x; t < nv; t += gridDim.x * 256u) {
    uint32_t coord[kMaxRank] = {};
    if (p.any_strided) {
      uint32_t rem = t;
#pragma unroll
      for (int d = kMaxRank - 1; d >= 1; --d) {
        if (d < p.rank) {
          const uint32_t q = fastdiv(rem, p.div[d]);
          coord[d] = rem - q * p.div[d].d;
          rem = q;
        }
      }
      coord[0] = rem;
    }
#pragma unroll
    for (int k = 0; k < kFusedMaxIn; ++k) {
      if (k < p.n_in) {
        const uint32_t* src = static_cast<const uint32_t*>(p.in[k]);
        const int mode = p.in_mode[k];
        uint32_t off = 0;
        if (mode == FM_CONTIG) {
          off = t * VEC;
        } else if (mode != FM_SCALAR) {
#pragma unroll
          for (int d = 0; d < kMaxRank; ++d)
            if (d < p.rank) off += coord[d] * (uint32_t)p.in_strides[k][d];
        }
        uint32_t v[VEC];
        if (VEC == 4 && (mode == FM_CONTIG || mode == FM_STRIDED_V)) {
          const u32x4 w = *reinterpret_cast<const u32x4*>(src + off);
#pragma unroll
          for (int e = 0; e < VEC; ++e) v[e] = w[e];
        } else if (VEC == 1 || mode == FM_SCALAR || mode == FM_STRIDED_B) {
          const uint32_t w = src[off];
#pragma unroll
          for (int e = 0; e < VEC; ++e) v[e] = w;
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e) v[e] = src[off + e * p.in_inner[k]];
        }
        rstore<VEC>(my + k * (256 * VEC), v);
      }
    }
    run_program<VEC, 0>(code, p.n_instr, my, seed, t * VEC, 1, 0xffffffffu, nullptr);
#pragma unroll
    for (int k = 0; k < kFusedMaxOut; ++k) {
      if (k < p.n_out) {
        uint32_t* dstp = static_cast<uint32_t*>(p.out[k]);
        uint32_t v[VEC];
        rload<VEC>(my + p.out_reg[k] * (256 * VEC), v);
        if (VEC == 4) {
          u32x4 w;
#pragma unroll
          for (int e = 0; e < VEC; ++e) w[e] = v[e];
          *reinterpret_cast<u32x4*>(dstp + t * VEC) = w;
        } else {
          dstp[t] = v[0];
        }
      }
    }
  }
}

// Row form: the iteration space is rows x D; TPR threads own a row (one wavefront as
// launched), 256 / TPR rows per block, each thread EPT elements (j = lane + e * TPR).
// Operand k of row r, column j is at rowoff_k(r) + j * in_inner[k], rowoff from the row's
// coordinates over the merged row dims (p.div / p.in_strides). Outputs flagged in
// out_row are per-row values, stored once per row at index r.
template <int TPR, int EPT>
__global__ __launch_bounds__(256) void k_fused_rows(const FusedProgram p, uint32_t nrows, uint32_t D) {
  extern __shared__ __attribute__((aligned(16))) uint32_t regs[];   // 4 doubles of partials, then registers
  double* part = reinterpret_cast<double*>(regs);
  uint32_t* const my = regs + 16 + threadIdx.x * EPT;
  constexpr int RPB = 256 / TPR;
  const uint32_t seed = p.seed ? (uint32_t)*p.seed : 0u;
  const ConstCode code = (ConstCode)(uintptr_t)p.code;
  const uint32_t lane = threadIdx.x % TPR;
  // Every thread runs every iteration (uniform trip count), so barriers inside
  // FO_ROWSUM (TPR > 64) are reached by the whole block; threads of rows past the end
  // compute on zeros and store nothing.
  for (uint32_t rb = blockIdx.x * RPB; rb < nrows; rb += gridDim.x * RPB) {
    const uint32_t r = rb + threadIdx.x / TPR;
    const bool live_row = r < nrows;
    uint32_t live = 0;
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      if (live_row && lane + e * TPR < D) live |= 1u << e;
    uint32_t coord[kMaxRank] = {};
    {
      uint32_t rem = live_row ? r : 0u;
#pragma unroll
      for (int d = kMaxRank - 1; d >= 1; --d) {
        if (d < p.rank) {
          const uint32_t q = fastdiv(rem, p.div[d]);
          coord[d] = rem - q * p.div[d].d;
          rem = q;
        }
      }
      coord[0] = rem;
    }
#pragma unroll
    for (int k = 0; k < kFusedMaxIn; ++k) {
      if (k < p.n_in) {
        const uint32_t* src = static_cast<const uint32_t*>(p.in[k]);
        uint32_t off = 0;
#pragma unroll
        for (int d = 0; d < kMaxRank; ++d)
          if (d < p.rank) off += coord[d] * (uint32_t)p.in_strides[k][d];
        const uint32_t cs = (uint32_t)p.in_inner[k];
        uint32_t v[EPT];
#pragma unroll
        for (int e = 0; e < EPT; ++e) v[e] = ((live >> e) & 1u) ? src[off + (lane + e * TPR) * cs] : 0u;
        rstore<EPT>(my + k * (256 * EPT), v);
      }
    }
    run_program<EPT, TPR>(code, p.n_instr, my, seed, r * D + lane, TPR, live, part, live_row ? r % D : 0u);
#pragma unroll
    for (int k = 0; k < kFusedMaxOut; ++k) {
      if (k < p.n_out) {
        uint32_t* dstp = static_cast<uint32_t*>(p.out[k]);
        uint32_t v[EPT];
        rload<EPT>(my + p.out_reg[k] * (256 * EPT), v);
        if (p.out_row[k]) {
          if (live_row && lane == 0) dstp[r] = v[0];
        } else {
#pragma unroll
          for (int e = 0; e < EPT; ++e)
            if ((live >> e) & 1u) dstp[r * D + lane + e * TPR] = v[e];
        }
      }
    }
  }
}

}  // namespace

void fused(const FusedProgram& prog, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  if (prog.row_d > 0) {
    // n = number of rows
    const int D = prog.row_d;
    // One wavefront per row (reductions are wavefront butterflies, no block barriers),
    // four rows per block, ceil(D / 64) elements per lane.
    const int ept = D <= 64 ? 1 : (D <= 128 ? 2 : (D <= 256 ? 4 : (D <= 512 ? 8 : 16)));
    int64_t b = (n + 3) / 4;
    if (b > 16384) b = 16384;
    const size_t lds = 64 + (size_t)prog.nregs * ept * 256 * 4;   // 16 words of partials first
    if (ept == 1) klaunch(k_fused_rows<64, 1>, (int)b, 256, lds, st, prog, (uint32_t)n, (uint32_t)D);
    else if (ept == 2) klaunch(k_fused_rows<64, 2>, (int)b, 256, lds, st, prog, (uint32_t)n, (uint32_t)D);
    else if (ept == 4) klaunch(k_fused_rows<64, 4>, (int)b, 256, lds, st, prog, (uint32_t)n, (uint32_t)D);
    else if (ept == 8) klaunch(k_fused_rows<64, 8>, (int)b, 256, lds, st, prog, (uint32_t)n, (uint32_t)D);
    else klaunch(k_fused_rows<64, 16>, (int)b, 256, lds, st, prog, (uint32_t)n, (uint32_t)D);
    return;
  }
  int64_t b = (n + 255) / 256;
  if (b > 16384) b = 16384;
  // LDS holds only the registers the program uses.
  const size_t lds = (size_t)prog.nregs * prog.vec * 256 * 4;
  if (prog.vec == 4) klaunch(k_fused<4>, (int)b, 256, lds, st, prog, (uint32_t)n);
  else klaunch(k_fused<1>, (int)b, 256, lds, st, prog, (uint32_t)n);
}

}  // namespace tgk
