// Element arithmetic of the fused groups: one definition of every opcode's bits, shared
// by the ahead-of-time group interpreter (k_fused.hip) and the kernels generated per
// group at run time (jit.cpp compiles them with hipRTC, which reads this file as text,
// so it includes nothing under hipRTC and needs no host code).
//
// Every value is a 32-bit pattern: an f32, or an i32 (the `i32` and `bool` IR dtypes).
// Arithmetic follows the reference evaluator (test/_eval.ts): f64 operations rounded once
// to the result dtype, JS semantics for min / max / sign / ToInt32, and the reference's
// erf and dropout hash. Compile with -ffp-contract=off.
#ifndef TG_FUSED_DEV_H
#define TG_FUSED_DEV_H
#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cmath>
#endif

namespace tgk {

// dtype codes for element-wise operands
enum { DT_F32 = 0, DT_I32 = 1 };

// Opcodes FO_FADD .. FO_COPY are the inexpensive forms (f32 operands and result where
// typed); the rest are general forms (mixed i32 / f32 typing, comparisons, f64
// transcendentals, dropout) and the row-only reductions.
enum FusedOp {
  FO_FADD, FO_FSUB, FO_FMUL, FO_FDIV, FO_MULS, FO_ADDS, FO_SQRT, FO_NEG, FO_ABS, FO_RELU, FO_RELU_GRAD,
  FO_WHERE, FO_COPY,
  FO_ADD, FO_SUB, FO_MUL, FO_DIV, FO_MIN, FO_MAX, FO_LESS, FO_GREATER,
  FO_RSQRT, FO_LOG, FO_EXP, FO_TANH, FO_SIGMOID, FO_ERF, FO_SIN, FO_COS, FO_DROPOUT,
  FO_ROWSUM,          // row form only: dst = f32(sum over the row of a, in f64, / imm)
  FO_SOFTMAX_CAUSAL,  // row form only: causal softmax of row q = row % D (q + 1 leading entries)
  FO_LOG_SOFTMAX,     // row form only
  FO_ONEHOT           // row form only: dst = (i32 a == column) ? one : 0 (1.0f for f32 results, 1 for i32)
};

constexpr int kFusedMaxIn = 12;
constexpr int kFusedMaxOut = 8;

// Kernel argument of a generated group kernel: operand and output base pointers, and the
// per-step PRNG seed tensor (null without dropout). Shapes and strides are compiled in.
struct JitArgs {
  const void* in[kFusedMaxIn];
  void* out[kFusedMaxOut];
  const int* seed;
};
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ unsigned fbits(float x) { return __float_as_uint(x); }
__device__ __forceinline__ float bitsf(unsigned x) { return __uint_as_float(x); }

// ---- wavefront butterflies -------------------------------------------------------------------
// Sum or max over the 64 lanes of a wavefront, every lane receiving the result, as the
// butterfly over lane distances 32, 16, 8, 4, 2, 1: at distance d each lane combines its
// value with lane ^ d's. Both lanes of a pair combine the same two values with a commutative
// operation, so afterwards every lane holds the same bits as lane ^ d, and cheaper moves than
// an xor shuffle through LDS give the same result bit for bit: permlane32_swap and
// permlane16_swap hand each lane its own value and its partner's (in either order) for 32
// and 16; DPP row rotations by 8 and 4 within a 16-lane row for 8 and 4 (after distance 8
// a row's values repeat with period 8, so the rotation by 4 brings lane ^ 4's value); DPP
// quad permutations for 2 and 1.
constexpr int kDppRor8 = 0x128, kDppRor4 = 0x124, kDppQuadXor2 = 0x4E, kDppQuadXor1 = 0xB1;

template <int Ctrl> __device__ __forceinline__ unsigned dpp_u32(unsigned v) {
  return (unsigned)__builtin_amdgcn_mov_dpp((int)v, Ctrl, 0xF, 0xF, false);
}
template <int Ctrl> __device__ __forceinline__ float dpp_move(float v) { return bitsf(dpp_u32<Ctrl>(fbits(v))); }
template <int Ctrl> __device__ __forceinline__ double dpp_move(double v) {
  const unsigned long long u = (unsigned long long)__double_as_longlong(v);
  const unsigned long long lo = dpp_u32<Ctrl>((unsigned)u), hi = dpp_u32<Ctrl>((unsigned)(u >> 32));
  return __longlong_as_double((long long)((hi << 32) | lo));
}
// {a, b} = {own value, value of lane ^ 32} (Half false) or lane ^ 16 (Half true)
template <bool Half> __device__ __forceinline__ void lane_pair(float v, float& a, float& b) {
  const auto p = Half ? __builtin_amdgcn_permlane16_swap(fbits(v), fbits(v), false, false)
                      : __builtin_amdgcn_permlane32_swap(fbits(v), fbits(v), false, false);
  a = bitsf(p[0]);
  b = bitsf(p[1]);
}
template <bool Half> __device__ __forceinline__ void lane_pair(double v, double& a, double& b) {
  const unsigned long long u = (unsigned long long)__double_as_longlong(v);
  const unsigned lo = (unsigned)u, hi = (unsigned)(u >> 32);
  const auto pl = Half ? __builtin_amdgcn_permlane16_swap(lo, lo, false, false)
                       : __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
  const auto ph = Half ? __builtin_amdgcn_permlane16_swap(hi, hi, false, false)
                       : __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
  a = __longlong_as_double((long long)(((unsigned long long)ph[0] << 32) | pl[0]));
  b = __longlong_as_double((long long)(((unsigned long long)ph[1] << 32) | pl[1]));
}
struct WaveAdd {
  template <class T> __device__ __forceinline__ T operator()(T x, T y) const { return x + y; }
};
struct WaveMax {
  __device__ __forceinline__ float operator()(float x, float y) const { return fmaxf(x, y); }
};
template <class T, class Op> __device__ __forceinline__ T wave_allreduce(T v, Op op) {
  T a, b;
  lane_pair<false>(v, a, b);
  v = op(a, b);
  lane_pair<true>(v, a, b);
  v = op(a, b);
  v = op(v, dpp_move<kDppRor8>(v));
  v = op(v, dpp_move<kDppRor4>(v));
  v = op(v, dpp_move<kDppQuadXor2>(v));
  v = op(v, dpp_move<kDppQuadXor1>(v));
  return v;
}
__device__ __forceinline__ double wave_allsum(double v) { return wave_allreduce(v, WaveAdd()); }
__device__ __forceinline__ float wave_allsum(float v) { return wave_allreduce(v, WaveAdd()); }
__device__ __forceinline__ float wave_allmax(float v) { return wave_allreduce(v, WaveMax()); }

__device__ __forceinline__ double js_max(double a, double b) {
  if (isnan(a) || isnan(b)) return __longlong_as_double(0x7ff8000000000000LL);
  if (a == 0.0 && b == 0.0) return (signbit(a) && signbit(b)) ? -0.0 : 0.0;
  return a > b ? a : b;
}
__device__ __forceinline__ double js_min(double a, double b) {
  if (isnan(a) || isnan(b)) return __longlong_as_double(0x7ff8000000000000LL);
  if (a == 0.0 && b == 0.0) return (signbit(a) || signbit(b)) ? -0.0 : 0.0;
  return a < b ? a : b;
}
__device__ __forceinline__ double js_sign(double x) {
  if (isnan(x)) return x;
  return x > 0 ? 1.0 : (x < 0 ? -1.0 : x);
}
// ECMAScript ToInt32.
__device__ __forceinline__ int to_int32(double x) {
  if (!isfinite(x)) return 0;
  double m = fmod(trunc(x), 4294967296.0);
  if (m < 0) m += 4294967296.0;
  return (int)(unsigned)m;
}
// t mod 2^32 of a non-negative integer-valued double below 2^64: t * 2^-32 and its floor
// are exact, and so is t - q * 2^32 (it fits 32 bits); four f64 operations instead of a
// general double -> u64 conversion.
__device__ __forceinline__ unsigned mod32_f64(double t) {
  const double q = floor(__dmul_rn(t, 2.3283064365386963e-10));
  return (unsigned)__fma_rn(-q, 4294967296.0, t);
}

// The reference's PCG-style hash with its f64 multiply-adds (products below 2^53 are exact
// in f64, larger ones round to integers; the casts take the value modulo 2^32).
__device__ __forceinline__ unsigned pcg_f64(unsigned seed, unsigned sc, unsigned idx) {
  unsigned h = seed ^ sc ^ idx;
  double t = __dadd_rn(__dmul_rn((double)h, 747796405.0), 2891336453.0);
  h = mod32_f64(t);
  unsigned x = h ^ (h >> ((h >> 28) + 4));
  double t2 = __dmul_rn((double)x, 277803737.0);
  h = mod32_f64(t2);
  return h ^ (h >> 22);
}

__device__ __forceinline__ double num(unsigned x, int dt) { return dt == DT_F32 ? (double)bitsf(x) : (double)(int)x; }
__device__ __forceinline__ unsigned from_num(double v, int dt) {
  return dt == DT_F32 ? fbits((float)v) : (unsigned)to_int32(v);
}

// Abramowitz & Stegun 7.1.26, the reference's erf (test/_eval.ts:193-198).
__device__ __forceinline__ float erf_as(float xf) {
  const double v = xf;
  const double sg = js_sign(v), av = fabs(v);
  const double t = 1.0 / (1.0 + 0.3275911 * av);
  const double pl = t * (0.254829592 + t * (-0.284496736 + t * (1.421413741 + t * (-1.453152027 + t * 1.061405429))));
  return (float)(sg * (1.0 - pl * exp(-av * av)));
}

// Inverted dropout of one element: keep with probability 1 - p, scaled by 1 / (1 - p)
// (test/_eval.ts dropout; u = hash / 2^32).
__device__ __forceinline__ unsigned dropout_bits(unsigned x, unsigned seed, unsigned salt, double p, double scale,
                                                 unsigned elem) {
  const unsigned hh = pcg_f64(seed, salt, elem);
  const double u = (double)hh / 4294967296.0;
  return fbits((float)((double)bitsf(x) * (u >= p ? scale : 0.0)));
}

// One element of opcode `op` (every opcode but FO_WHERE and the row-only ones). With a
// constant opcode and dtypes, inlining leaves only that opcode's arithmetic.
__device__ __forceinline__ unsigned op_eval(int op, unsigned x, unsigned y, int ta, int tb, int dt, double imm,
                                            double imm2, unsigned salt, unsigned seed, unsigned elem) {
  switch (op) {
    // f32 +, -, *, /: the correctly rounded f32 operation equals computing in f64 and
    // rounding once.
    case FO_FADD: return fbits(bitsf(x) + bitsf(y));
    case FO_FSUB: return fbits(bitsf(x) - bitsf(y));
    case FO_FMUL: return fbits(bitsf(x) * bitsf(y));
    case FO_FDIV: return fbits(bitsf(x) / bitsf(y));
    case FO_MULS: return fbits((float)(num(x, ta) * imm));
    case FO_ADDS: return fbits((float)(num(x, ta) + imm));
    // f64 sqrt rounded once to f32 is the correctly rounded f32 square root.
    case FO_SQRT: return fbits((float)sqrt((double)bitsf(x)));
    case FO_NEG: return x ^ 0x80000000u;
    case FO_ABS: return x & 0x7fffffffu;
    // max(x, 0) with JS semantics: NaN stays NaN, -0 becomes +0.
    case FO_RELU: return bitsf(x) != bitsf(x) ? 0x7fc00000u : (bitsf(x) > 0.0f ? x : 0u);
    case FO_RELU_GRAD: return bitsf(x) > 0.0f ? y : 0u;
    case FO_COPY: return x;
    case FO_ADD: return from_num(num(x, ta) + num(y, tb), dt);
    case FO_SUB: return from_num(num(x, ta) - num(y, tb), dt);
    case FO_MUL: return from_num(num(x, ta) * num(y, tb), dt);
    case FO_DIV: return from_num(num(x, ta) / num(y, tb), dt);
    case FO_MIN: return from_num(js_min(num(x, ta), num(y, tb)), dt);
    case FO_MAX: return from_num(js_max(num(x, ta), num(y, tb)), dt);
    case FO_LESS: return num(x, ta) < num(y, tb) ? 1u : 0u;
    case FO_GREATER: return num(x, ta) > num(y, tb) ? 1u : 0u;
    case FO_RSQRT: return fbits((float)(1.0 / sqrt((double)bitsf(x))));
    case FO_LOG: return fbits((float)log((double)bitsf(x)));
    case FO_EXP: return fbits((float)exp((double)bitsf(x)));
    case FO_TANH: return fbits((float)tanh((double)bitsf(x)));
    case FO_SIGMOID: return fbits((float)(0.5 + 0.5 * tanh(0.5 * (double)bitsf(x))));
    case FO_ERF: return fbits(erf_as(bitsf(x)));
    case FO_SIN: return fbits((float)sin((double)bitsf(x)));
    case FO_COS: return fbits((float)cos((double)bitsf(x)));
    case FO_DROPOUT: return dropout_bits(x, seed, salt, imm, imm2, elem);
    default: return 0u;
  }
}

}  // namespace tgk

#endif  // TG_FUSED_DEV_H
