// Element-wise, data-movement and stochastic kernels for gfx950.
//
// Arithmetic follows the reference evaluator's numerics (test/_eval.ts:133-203): each
// op computes in f64 on the f32 operands and rounds once when stored, so results are
// identical to the CPU evaluation. These kernels are HBM-bound; f64 ALU work is far
// below what the memory system delivers per byte. Built with -ffp-contract=off.
//
// Launch shape: 256-thread blocks, grid-stride loops, grid capped at 8 blocks per CU
// for 256 CUs so that large tensors are covered by resident waves.
#include "kernels.h"

#include <cmath>
#include <cstring>
#include <stdexcept>

namespace tgk {
namespace {

constexpr int kThreads = 256;

inline int grid_for(int64_t n) {
  int64_t b = (n + kThreads - 1) / kThreads;
  if (b > 2048) b = 2048;
  if (b < 1) b = 1;
  return (int)b;
}

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

// JS ToInt32 for an f64 stored into an Int32Array.
__device__ __forceinline__ int32_t to_int32(double x) {
  if (!isfinite(x)) return 0;
  double t = trunc(x);
  double m = fmod(t, 4294967296.0);
  if (m < 0) m += 4294967296.0;
  return (int32_t)(uint32_t)m;
}

__device__ __forceinline__ double load_num(const void* p, int dt, int64_t i) {
  return dt == DT_F32 ? (double)static_cast<const float*>(p)[i] : (double)static_cast<const int32_t*>(p)[i];
}

__device__ __forceinline__ void store_num(void* p, int dt, int64_t i, double x) {
  if (dt == DT_F32) static_cast<float*>(p)[i] = (float)x;
  else static_cast<int32_t*>(p)[i] = to_int32(x);
}

// Decompose flat index i over sp.dims and accumulate up to three operand offsets.
template <int NOPS>
__device__ __forceinline__ void offsets(const Strided& sp, int64_t i, int64_t* o) {
  o[0] = 0;
  if (NOPS > 1) o[1] = 0;
  if (NOPS > 2) o[2] = 0;
  for (int d = sp.rank - 1; d >= 0; --d) {
    int64_t dim = sp.dims[d];
    int64_t c = i % dim;
    i /= dim;
    o[0] += c * sp.s0[d];
    if (NOPS > 1) o[1] += c * sp.s1[d];
    if (NOPS > 2) o[2] += c * sp.s2[d];
  }
}

__global__ void k_binary(int op, const void* __restrict__ a, int adt, const void* __restrict__ b, int bdt,
                         void* __restrict__ out, int odt, Strided sp, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t o[2];
    offsets<2>(sp, i, o);
    double x = load_num(a, adt, o[0]), y = load_num(b, bdt, o[1]);
    double r;
    switch (op) {
      case B_ADD: r = x + y; break;
      case B_SUB: r = x - y; break;
      case B_MUL: r = x * y; break;
      case B_DIV: r = x / y; break;
      case B_MIN: r = js_min(x, y); break;
      case B_MAX: r = js_max(x, y); break;
      case B_LESS: r = x < y ? 1.0 : 0.0; break;
      default: r = x > y ? 1.0 : 0.0; break;
    }
    store_num(out, odt, i, r);
  }
}

// Same-shape fast path: a, b and out all contiguous with identical shape.
__global__ void k_binary_flat(int op, const float* __restrict__ a, const float* __restrict__ b,
                              float* __restrict__ out, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    double x = a[i], y = b[i], r;
    switch (op) {
      case B_ADD: r = x + y; break;
      case B_SUB: r = x - y; break;
      case B_MUL: r = x * y; break;
      case B_DIV: r = x / y; break;
      case B_MIN: r = js_min(x, y); break;
      default: r = js_max(x, y); break;
    }
    out[i] = (float)r;
  }
}

__global__ void k_scalar(bool mul, const void* __restrict__ a, int adt, double s, float* __restrict__ out, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    double x = load_num(a, adt, i);
    out[i] = (float)(mul ? x * s : x + s);
  }
}

__device__ __forceinline__ double js_sign(double x) {
  if (isnan(x)) return x;
  if (x > 0) return 1.0;
  if (x < 0) return -1.0;
  return x;
}

// Abramowitz & Stegun 7.1.26, the reference's erf (_eval.ts:193-198).
__device__ __forceinline__ double erf_as(double x) {
  double s = js_sign(x), ax = fabs(x);
  double t = 1.0 / (1.0 + 0.3275911 * ax);
  double p = t * (0.254829592 + t * (-0.284496736 + t * (1.421413741 + t * (-1.453152027 + t * 1.061405429))));
  return s * (1.0 - p * exp(-ax * ax));
}

__global__ void k_unary(int op, const float* __restrict__ a, float* __restrict__ out, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    double x = a[i], r;
    switch (op) {
      case U_SQRT: r = sqrt(x); break;
      case U_RSQRT: r = 1.0 / sqrt(x); break;
      case U_LOG: r = log(x); break;
      case U_EXP: r = exp(x); break;
      case U_RELU: r = js_max(x, 0.0); break;
      case U_NEG: r = -x; break;
      case U_ABS: r = fabs(x); break;
      case U_TANH: r = tanh(x); break;
      case U_SIGMOID: r = 0.5 + 0.5 * tanh(0.5 * x); break;
      case U_ERF: r = erf_as(x); break;
      case U_SIN: r = sin(x); break;
      default: r = cos(x); break;
    }
    out[i] = (float)r;
  }
}

__global__ void k_relu_grad(const float* __restrict__ x, const float* __restrict__ dy, float* __restrict__ out,
                            int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = x[i] > 0.0f ? dy[i] : 0.0f;
}

__global__ void k_where(const int32_t* __restrict__ c, const void* __restrict__ a, const void* __restrict__ b, int dt,
                        void* __restrict__ out, Strided sp, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t o[3];
    offsets<3>(sp, i, o);
    const uint32_t* src = (const uint32_t*)(c[o[0]] != 0 ? a : b);
    static_cast<uint32_t*>(out)[i] = src[c[o[0]] != 0 ? o[1] : o[2]];
  }
}

__global__ void k_where_causal(const float* __restrict__ a, float* __restrict__ out, int64_t total, int64_t D,
                               float fill) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t j = i % D, r = (i / D) % D;
    out[i] = j <= r ? a[i] : fill;
  }
}

__global__ void k_strided_copy(uint32_t* __restrict__ dst, const uint32_t* __restrict__ src, Strided sp, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t o[2];
    offsets<2>(sp, i, o);
    dst[o[0]] = src[o[1]];
  }
}

// 32-bit index form of strided_copy: merged dims, divisions by invariant multiplication,
// VEC consecutive elements per thread (VEC = 4: 128-bit loads and stores).
struct Copy32 {
  int rank;
  FastDiv fd[kMaxRank];
  int32_t sd[kMaxRank], ss[kMaxRank];   // innermost strides already scaled by VEC
};
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int VEC>
__global__ __launch_bounds__(256) void k_copy32(uint32_t* __restrict__ dst, const uint32_t* __restrict__ src, Copy32 c,
                                                uint32_t nv) {
  for (uint32_t t = blockIdx.x * 256u + threadIdx.x; t < nv; t += gridDim.x * 256u) {
    uint32_t rem = t, od = 0, os = 0;
#pragma unroll
    for (int d = kMaxRank - 1; d >= 0; --d) {
      if (d < c.rank) {
        uint32_t cd = rem;
        if (d > 0) {
          const uint32_t q = fastdiv(rem, c.fd[d]);
          cd = rem - q * c.fd[d].d;
          rem = q;
        }
        od += cd * (uint32_t)c.sd[d];
        os += cd * (uint32_t)c.ss[d];
      }
    }
    if (VEC == 4) *reinterpret_cast<u32x4*>(dst + od) = *reinterpret_cast<const u32x4*>(src + os);
    else dst[od] = src[os];
  }
}

// Output element t of a last-axis concatenation: row t / W, column c = t % W, taken from
// the input whose column range holds c. Consecutive threads write consecutive elements, so
// every output line is written whole by one launch.
// Four elements per thread and round (t, t + S, t + 2S, t + 3S for the grid's stride S),
// their loads issued before any store.
__global__ __launch_bounds__(256) void k_concat_last(uint32_t* __restrict__ dst, const ConcatLast c, FastDiv fw,
                                                     uint32_t total) {
  const uint32_t S = gridDim.x * 256u;
  for (uint32_t t0 = blockIdx.x * 256u + threadIdx.x; t0 < total; t0 += 4 * S) {
    uint32_t v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t t = min(t0 + u * S, total - 1);   // past the end: the last element again
      const uint32_t r = fastdiv(t, fw), col = t - r * fw.d;
      // the input holding column col: a uniform loop over the inputs with per-lane selects
      // (an array index that differs between lanes would place c in scratch memory)
      const uint32_t* sp = c.src[0];
      uint32_t lo = 0, hi = c.off[1];
#pragma unroll
      for (int j = 1; j < kConcatMax; ++j) {
        const bool in = j < c.n && col >= c.off[j];
        sp = in ? c.src[j] : sp;
        lo = in ? c.off[j] : lo;
        hi = in ? c.off[j + 1] : hi;
      }
      v[u] = sp[r * (hi - lo) + (col - lo)];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (t0 + u * S < total) dst[t0 + u * S] = v[u];
  }
}

__global__ void k_fill(uint32_t* __restrict__ dst, uint32_t bits, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = bits;
}

__global__ void k_arange(void* __restrict__ dst, int dt, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if (dt == DT_F32) static_cast<float*>(dst)[i] = (float)i;
    else static_cast<int32_t*>(dst)[i] = (int32_t)i;
  }
}

__global__ void k_one_hot(const int32_t* __restrict__ idx, int64_t total, int64_t depth, void* __restrict__ out, int dt) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    bool hit = idx[i / depth] == (int32_t)(i % depth);
    if (dt == DT_F32) static_cast<float*>(out)[i] = hit ? 1.0f : 0.0f;
    else static_cast<int32_t*>(out)[i] = hit ? 1 : 0;
  }
}

// The dropout / categorical hash exactly as the reference evaluator computes it
// (_eval.ts:568-571): both multiplies are IEEE f64 products (rounded above 2^53) taken
// modulo 2^32. The explicit _rn intrinsics rule out any fused multiply-add.
__device__ __forceinline__ uint32_t pcg_f64(uint32_t seed, uint32_t sc, uint32_t idx) {
  uint32_t h = seed ^ sc ^ idx;
  double t = __dadd_rn(__dmul_rn((double)h, 747796405.0), 2891336453.0);
  h = (uint32_t)(unsigned long long)t;
  uint32_t x = h ^ (h >> ((h >> 28) + 4));
  double t2 = __dmul_rn((double)x, 277803737.0);
  h = (uint32_t)(unsigned long long)t2;
  return h ^ (h >> 22);
}

__global__ void k_dropout(const float* __restrict__ a, float* __restrict__ out, int64_t n, const int32_t* seedp,
                          uint32_t sc, double p, double scale) {
  uint32_t seed = (uint32_t)*seedp;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    uint32_t h = pcg_f64(seed, sc, (uint32_t)i);
    double u = (double)h / 4294967296.0;
    double mask = u >= p ? scale : 0.0;
    out[i] = (float)((double)a[i] * mask);
  }
}

__global__ void k_randn(float* __restrict__ out, int64_t n, const int32_t* seedp, uint32_t sc) {
  uint32_t seed = (uint32_t)*seedp;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    uint32_t h1 = seed ^ sc ^ (uint32_t)i;
    h1 = h1 * 747796405u + 2891336453u;
    h1 = (h1 ^ (h1 >> ((h1 >> 28) + 4))) * 277803737u;
    h1 = h1 ^ (h1 >> 22);
    uint32_t h2 = h1 * 747796405u + 2891336453u;
    h2 = (h2 ^ (h2 >> ((h2 >> 28) + 4))) * 277803737u;
    h2 = h2 ^ (h2 >> 22);
    double u1 = fmax(1e-10, (double)h1 / 4294967296.0), u2 = (double)h2 / 4294967296.0;
    out[i] = (float)(sqrt(-2.0 * log(u1)) * cos(2.0 * M_PI * u2));
  }
}

__global__ void k_categorical(const float* __restrict__ a, int32_t* __restrict__ out, int64_t outer, int64_t D,
                              const int32_t* seedp, uint32_t sc) {
  uint32_t seed = (uint32_t)*seedp;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < outer; i += (int64_t)gridDim.x * blockDim.x) {
    double best = -INFINITY;
    int32_t bi = 0;
    for (int64_t j = 0; j < D; ++j) {
      uint32_t h = pcg_f64(seed, sc, (uint32_t)(i * D + j));
      double u = fmax(1e-10, (double)h / 4294967296.0);
      double v = (double)a[i * D + j] + (-log(-log(u)));
      if (v > best) { best = v; bi = (int32_t)j; }
    }
    out[i] = bi;
  }
}

}  // namespace

void binary(int op, const void* a, int a_dt, const void* b, int b_dt, void* out, int out_dt, const Strided& sp,
            int64_t n, hipStream_t st) {
  if (n <= 0) return;
  bool flat = op <= B_MAX && a_dt == DT_F32 && b_dt == DT_F32 && out_dt == DT_F32;
  if (flat) {
    int64_t c = 1;
    for (int d = sp.rank - 1; d >= 0; --d) {
      if (sp.s0[d] != c || sp.s1[d] != c) { flat = false; break; }
      c *= sp.dims[d];
    }
  }
  if (flat) {
    klaunch(k_binary_flat, grid_for(n), kThreads, 0, st, op, (const float*)a, (const float*)b, (float*)out, n);
  } else {
    klaunch(k_binary, grid_for(n), kThreads, 0, st, op, a, a_dt, b, b_dt, out, out_dt, sp, n);
  }
}

void scalar_op(bool mul, const void* a, int a_dt, double s, float* out, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  klaunch(k_scalar, grid_for(n), kThreads, 0, st, mul, a, a_dt, s, out, n);
}

void unary(int op, const float* a, float* out, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  klaunch(k_unary, grid_for(n), kThreads, 0, st, op, a, out, n);
}

void relu_grad(const float* x, const float* dy, float* out, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  klaunch(k_relu_grad, grid_for(n), kThreads, 0, st, x, dy, out, n);
}

void where(const int32_t* cond, const void* a, const void* b, int dt, void* out, const Strided& sp, int64_t n,
           hipStream_t st) {
  (void)dt;
  if (n <= 0) return;
  klaunch(k_where, grid_for(n), kThreads, 0, st, cond, a, b, dt, out, sp, n);
}

void where_causal(const float* a, float* out, int64_t outer, int64_t D, double fill, hipStream_t st) {
  int64_t total = outer * D * D;
  if (total <= 0) return;
  klaunch(k_where_causal, grid_for(total), kThreads, 0, st, a, out, total, D, (float)fill);
}

void concat_last(uint32_t* dst, const ConcatLast& c, int64_t rows, hipStream_t st) {
  if (c.n < 1 || c.n > kConcatMax) throw std::runtime_error("concat: input count out of range");
  const int64_t W = c.off[c.n], total = rows * W;
  if (total <= 0) return;
  if (total >= (int64_t(1) << 31)) throw std::runtime_error("concat: output too large for 32-bit indexing");
  int64_t b = (total + 1023) / 1024;
  if (b > 8192) b = 8192;
  klaunch(k_concat_last, (int)b, 256, 0, st, dst, c, make_fastdiv((uint32_t)W), (uint32_t)total);
}

void strided_copy(void* dst, const void* src, const Strided& sp, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  // Drop size-1 dims and merge dims contiguous in both operands.
  int64_t dd[kMaxRank], s0[kMaxRank], s1[kMaxRank];
  int r = 0;
  int64_t span0 = 0, span1 = 0;
  for (int d = 0; d < sp.rank; ++d) {
    if (sp.dims[d] == 1) continue;
    span0 += (sp.dims[d] - 1) * (sp.s0[d] < 0 ? -sp.s0[d] : sp.s0[d]);
    span1 += (sp.dims[d] - 1) * (sp.s1[d] < 0 ? -sp.s1[d] : sp.s1[d]);
    if (r > 0 && s0[r - 1] == sp.s0[d] * sp.dims[d] && s1[r - 1] == sp.s1[d] * sp.dims[d]) {
      dd[r - 1] *= sp.dims[d]; s0[r - 1] = sp.s0[d]; s1[r - 1] = sp.s1[d];
    } else {
      dd[r] = sp.dims[d]; s0[r] = sp.s0[d]; s1[r] = sp.s1[d]; ++r;
    }
  }
  bool small = n < (int64_t(1) << 31) && span0 < (int64_t(1) << 31) && span1 < (int64_t(1) << 31);
  for (int d = 0; d < r; ++d) if (s0[d] < 0 || s1[d] < 0) small = false;
  if (!small) {
    klaunch(k_strided_copy, grid_for(n), kThreads, 0, st, (uint32_t*)dst, (const uint32_t*)src, sp, n);
    return;
  }
  if (r == 0) { dd[0] = 1; s0[0] = s1[0] = 0; r = 1; }
  bool v4 = dd[r - 1] % 4 == 0 && s0[r - 1] == 1 && s1[r - 1] == 1 && ((uintptr_t)dst & 15) == 0 &&
            ((uintptr_t)src & 15) == 0;
  for (int d = 0; d < r - 1 && v4; ++d) v4 = s0[d] % 4 == 0 && s1[d] % 4 == 0;
  const int vec = v4 ? 4 : 1;
  Copy32 c{};
  c.rank = r;
  for (int d = 0; d < r; ++d) {
    c.fd[d] = make_fastdiv((uint32_t)(d == r - 1 ? dd[d] / vec : dd[d]));
    c.sd[d] = (int32_t)(d == r - 1 ? s0[d] * vec : s0[d]);
    c.ss[d] = (int32_t)(d == r - 1 ? s1[d] * vec : s1[d]);
  }
  const int64_t nv = n / vec;
  int64_t b = (nv + 255) / 256;
  if (b > 16384) b = 16384;
  if (vec == 4) klaunch(k_copy32<4>, (int)b, 256, 0, st, (uint32_t*)dst, (const uint32_t*)src, c, (uint32_t)nv);
  else klaunch(k_copy32<1>, (int)b, 256, 0, st, (uint32_t*)dst, (const uint32_t*)src, c, (uint32_t)nv);
}

void fill(void* dst, int dt, double value, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  uint32_t bits;
  if (dt == DT_F32) { float f = (float)value; memcpy(&bits, &f, 4); }
  else { int32_t v = (int32_t)value; memcpy(&bits, &v, 4); }
  klaunch(k_fill, grid_for(n), kThreads, 0, st, (uint32_t*)dst, bits, n);
}

void arange(void* dst, int dt, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  klaunch(k_arange, grid_for(n), kThreads, 0, st, dst, dt, n);
}

void one_hot(const int32_t* idx, int64_t rows, int64_t depth, void* out, int dt, hipStream_t st) {
  int64_t total = rows * depth;
  if (total <= 0) return;
  klaunch(k_one_hot, grid_for(total), kThreads, 0, st, idx, total, depth, out, dt);
}

void dropout(const float* a, float* out, int64_t n, const int32_t* seed, uint32_t salt_const, double p,
             hipStream_t st) {
  if (n <= 0) return;
  klaunch(k_dropout, grid_for(n), kThreads, 0, st, a, out, n, seed, salt_const, p, 1.0 / (1.0 - p));
}

void randn(float* out, int64_t n, const int32_t* seed, uint32_t salt_const, hipStream_t st) {
  if (n <= 0) return;
  klaunch(k_randn, grid_for(n), kThreads, 0, st, out, n, seed, salt_const);
}

void categorical(const float* a, int32_t* out, int64_t outer, int64_t D, const int32_t* seed, uint32_t salt_const,
                 hipStream_t st) {
  if (outer <= 0) return;
  klaunch(k_categorical, grid_for(outer), kThreads, 0, st, a, out, outer, D, seed, salt_const);
}

}  // namespace tgk
