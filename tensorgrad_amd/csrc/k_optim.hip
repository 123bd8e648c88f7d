// Fused multi-tensor optimizer for gfx950: one launch updates every parameter in place,
// replacing the reference's per-parameter kernels and writeback copies
// (src/codegen.ts:841-905, src/runtime.ts:354-356; SGD: the pointwise chain of
// src/sgd.ts:155-170). Gradient clipping and normalisation (src/grad.ts:110-172) add one
// deterministic sum-of-squares launch (two when both are set) ahead of it.
//
// Adam, per element, in f64 from the f32 operands, each result rounded to f32 once:
//   m' = b1*m + (1-b1)*g
//   v' = b2*v + ((1-b2)*g)*g
//   p' = shrink*p - (lrt*m') / (sqrt(v') + eps)       (m', v' as stored f32 values)
// which is the numeric convention of the CPU oracle, so updates are bit-identical to it.
// SGD restates the IR ops one by one, each rounded to f32 as the evaluator stores it:
//   e  = f32(g + f32(p * wd))            (decayed parameters)
//   v' = f32(f32(v * mu) + e)            (momentum)
//   u  = f32(e + f32(v' * mu)) | v' | e  (Nesterov | momentum | plain)
//   p' = f32(p - f32(lr * u))
// Gradient transforms first: g = f32(g / norm) (normalizeGrads), then g = f32(g * scale)
// (clipGradNorm), the IR's div and mul by a broadcast scalar.
// Every operation is an explicitly rounded intrinsic: no contraction into FMA.
// HBM traffic: Adam 28 bytes per parameter (read p, g, m, v; write p, m, v); SGD 12, 20
// with momentum; a norm launch reads each gradient once (4 bytes per element).
#include "kernels.h"

namespace tgk {
namespace {

constexpr int kThreads = 256;
static_assert(kAdamChunk == kThreads * 8, "a thread updates two float4 of a full chunk");

enum { kSgdNesterov = 1, kSgdDecay = 2, kSgdMomentum = 4 };

struct Upd { float p, m, v; };

__device__ __forceinline__ Upd adam_elem(float gf, float mf0, float vf0, float pf, double lrt, double shrink,
                                         const AdamHyper& h) {
  const double g = (double)gf;
  const double m = __dadd_rn(__dmul_rn(h.beta1, (double)mf0), __dmul_rn(h.one_minus_beta1, g));
  const double v = __dadd_rn(__dmul_rn(h.beta2, (double)vf0), __dmul_rn(__dmul_rn(h.one_minus_beta2, g), g));
  const float mf = (float)m, vf = (float)v;
  const double upd = __ddiv_rn(__dmul_rn(lrt, (double)mf), __dadd_rn(__dsqrt_rn((double)vf), h.eps));
  return {(float)__dsub_rn(__dmul_rn(shrink, (double)pf), upd), mf, vf};
}

__device__ __forceinline__ Upd sgd_elem(float g, float v0, float p, double lr, double wd, double mu, int flags) {
  float e = g;
  if (flags & kSgdDecay) e = (float)__dadd_rn((double)g, (double)(float)__dmul_rn((double)p, wd));
  float u = e, vn = v0;
  if (flags & kSgdMomentum) {
    vn = (float)__dadd_rn((double)(float)__dmul_rn((double)v0, mu), (double)e);
    u = (flags & kSgdNesterov) ? (float)__dadd_rn((double)e, (double)(float)__dmul_rn((double)vn, mu)) : vn;
  }
  return {(float)__dsub_rn((double)p, (double)(float)__dmul_rn(lr, (double)u)), vn, 0.0f};
}

// The gradient transforms of a chunk: divide (normalise), then multiply (clip).
struct GradXf {
  bool div, mul;
  double d, m;
  __device__ __forceinline__ float operator()(float g) const {
    if (div) g = (float)__ddiv_rn((double)g, d);
    if (mul) g = (float)__dmul_rn((double)g, m);
    return g;
  }
};

__device__ __forceinline__ GradXf chunk_xf(const AdamChunk& k, const float* vals) {
  GradXf x{k.gdiv >= 0, k.gmul >= 0, 1.0, 1.0};
  if (x.div) x.d = (double)vals[k.gdiv];
  if (x.mul) x.m = (double)vals[k.gmul];
  return x;
}

// Block b updates chunks b, b + grid, ...: one descriptor load per chunk, then every
// operand of a full, 16-byte aligned chunk as two float4 per thread, all loads issued
// before the arithmetic; partial or unaligned chunks go element by element.
template <bool kSgd>
__global__ __launch_bounds__(kThreads) void k_opt_chunks(const AdamChunk* __restrict__ cs, int64_t nchunks,
                                                         const float* __restrict__ lrp, AdamHyper h,
                                                         const float* __restrict__ vals) {
  const double lr = (double)*lrp;
  for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const AdamChunk k = cs[c];
    const GradXf xf = chunk_xf(k, vals);
    const double shrink = !kSgd && k.shrink_ptr ? (double)*k.shrink_ptr : k.shrink;
    const int flags = k.flags;
    float* __restrict__ P = k.p;
    float* __restrict__ M = k.m;
    float* __restrict__ V = k.v;
    const float* __restrict__ G = k.g;
    const bool has_m = !kSgd || (flags & kSgdMomentum);
    const bool vec = k.n == kAdamChunk &&
                     ((reinterpret_cast<uintptr_t>(P) | reinterpret_cast<uintptr_t>(G) |
                       (has_m ? reinterpret_cast<uintptr_t>(M) : 0) | (kSgd ? 0 : reinterpret_cast<uintptr_t>(V))) &
                      15) == 0;
    if (vec) {
      float4 g[2], m[2], v[2], p[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int q = threadIdx.x + u * kThreads;
        g[u] = reinterpret_cast<const float4*>(G)[q];
        p[u] = reinterpret_cast<const float4*>(P)[q];
        m[u] = has_m ? reinterpret_cast<const float4*>(M)[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        if (!kSgd) v[u] = reinterpret_cast<const float4*>(V)[q];
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int q = threadIdx.x + u * kThreads;
        const float gx = xf(g[u].x), gy = xf(g[u].y), gz = xf(g[u].z), gw = xf(g[u].w);
        if (kSgd) {
          const Upd a = sgd_elem(gx, m[u].x, p[u].x, lr, shrink, k.mom, flags);
          const Upd b = sgd_elem(gy, m[u].y, p[u].y, lr, shrink, k.mom, flags);
          const Upd d = sgd_elem(gz, m[u].z, p[u].z, lr, shrink, k.mom, flags);
          const Upd e = sgd_elem(gw, m[u].w, p[u].w, lr, shrink, k.mom, flags);
          reinterpret_cast<float4*>(P)[q] = make_float4(a.p, b.p, d.p, e.p);
          if (has_m) reinterpret_cast<float4*>(M)[q] = make_float4(a.m, b.m, d.m, e.m);
        } else {
          const Upd a = adam_elem(gx, m[u].x, v[u].x, p[u].x, lr, shrink, h);
          const Upd b = adam_elem(gy, m[u].y, v[u].y, p[u].y, lr, shrink, h);
          const Upd d = adam_elem(gz, m[u].z, v[u].z, p[u].z, lr, shrink, h);
          const Upd e = adam_elem(gw, m[u].w, v[u].w, p[u].w, lr, shrink, h);
          reinterpret_cast<float4*>(P)[q] = make_float4(a.p, b.p, d.p, e.p);
          reinterpret_cast<float4*>(M)[q] = make_float4(a.m, b.m, d.m, e.m);
          reinterpret_cast<float4*>(V)[q] = make_float4(a.v, b.v, d.v, e.v);
        }
      }
    } else {
      for (int64_t i = threadIdx.x; i < k.n; i += kThreads) {
        const float g = xf(G[i]);
        if (kSgd) {
          const Upd a = sgd_elem(g, has_m ? M[i] : 0.0f, P[i], lr, shrink, k.mom, flags);
          P[i] = a.p;
          if (has_m) M[i] = a.m;
        } else {
          const Upd a = adam_elem(g, M[i], V[i], P[i], lr, shrink, h);
          P[i] = a.p;
          M[i] = a.m;
          V[i] = a.v;
        }
      }
    }
  }
}

// f32(x * x) of a (possibly normalised) gradient element, as the evaluator's mul stores it.
__device__ __forceinline__ double sq_term(float x, bool pre, double d) {
  if (pre) x = (float)__ddiv_rn((double)x, d);
  return (double)(float)__dmul_rn((double)x, (double)x);
}

constexpr int kProgWindow = 512;   // scalar instructions staged in LDS at a time

// A block's f64 sum of one value per thread in a fixed order: wave butterflies, then the
// wave sums in order. Every thread gets the result.
__device__ __forceinline__ double block_sum(double v, double* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_allsum(v);
  __syncthreads();   // earlier readers of red are done
  if (lane == 0) red[w] = v;
  __syncthreads();
  double s = red[0];
#pragma unroll
  for (int i = 1; i < kThreads / 64; ++i) s += red[i];
  return s;
}

// One block per chunk of up to kNormChunk elements: thread t sums its (up to) 32 elements
// in order (eight float4, all loads issued first), the block sum gives the chunk's f64
// partial. The last block to finish a sum's chunks adds their partials (thread t over
// chunks t, t + 256, ... in order, then block_sum), rounds the sum to f32 into the value
// array and counts the sum in; the block finishing the last sum stages the value array
// and the program in LDS and runs the program on lane 0 of its first wave, with the
// opcode and operand indices made wave-uniform (readfirstlane) so that only the taken
// case executes. Partials, sums and counters cross blocks as device-scope atomics
// (coherent across the XCDs' L2 caches without a device-scope fence).
static_assert(kNormChunk == kThreads * 32, "a thread sums eight float4 of a full chunk");

__global__ __launch_bounds__(kThreads) void k_grad_norms(NormLaunch a) {
  __shared__ double red[kThreads / 64];
  __shared__ float sv[kNormMaxVals];
  __shared__ ScalarInstr sp[kProgWindow];
  __shared__ int flag;
  const SqChunk k = a.chunks[blockIdx.x];
  {
    const bool pre = k.pre >= 0;
    const double d = pre ? (double)a.vals[k.pre] : 1.0;
    double s = 0.0;
    if (k.n == kNormChunk && (reinterpret_cast<uintptr_t>(k.g) & 15) == 0) {
      float4 x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = reinterpret_cast<const float4*>(k.g)[threadIdx.x + u * kThreads];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        s += sq_term(x[u].x, pre, d);
        s += sq_term(x[u].y, pre, d);
        s += sq_term(x[u].z, pre, d);
        s += sq_term(x[u].w, pre, d);
      }
    } else {
      for (int64_t i = threadIdx.x; i < k.n; i += kThreads) s += sq_term(k.g[i], pre, d);
    }
    s = block_sum(s, red);
    if (threadIdx.x == 0) {
      __hip_atomic_store(&a.part[blockIdx.x], s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
      const unsigned nch = (unsigned)(a.slot_first[k.slot + 1] - a.slot_first[k.slot]);
      flag = __hip_atomic_fetch_add(&a.counters[k.slot], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nch - 1;
    }
    __syncthreads();
    if (!flag) return;
  }
  {
    const int c0 = a.slot_first[k.slot], c1 = a.slot_first[k.slot + 1];
    double t = 0.0;
    for (int c = c0 + (int)threadIdx.x; c < c1; c += kThreads)
      t += __hip_atomic_load(&a.part[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    t = block_sum(t, red);
    if (threadIdx.x == 0) {
      const float v = (float)t;
      __hip_atomic_store(reinterpret_cast<unsigned*>(&a.vals[a.slot_val[k.slot]]), __float_as_uint(v), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&a.counters[k.slot], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
      flag = __hip_atomic_fetch_add(&a.counters[a.nslots], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (unsigned)(a.nslots - 1);
    }
    __syncthreads();
    if (!flag) return;
  }
  for (int i = threadIdx.x; i < a.nvals; i += kThreads)
    sv[i] = __uint_as_float(__hip_atomic_load(reinterpret_cast<const unsigned*>(&a.vals[i]), __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT));
  for (int w0 = 0; w0 < a.nprog; w0 += kProgWindow) {
    const int nw = min(kProgWindow, a.nprog - w0);
    for (int i = threadIdx.x; i < nw; i += kThreads) sp[i] = a.prog[w0 + i];
    __syncthreads();
    if (threadIdx.x < 64) {
      // the whole first wave walks the program (so branches on the opcode are uniform);
      // lane 0 alone stores
      for (int i = 0; i < nw; ++i) {
        const int op = __builtin_amdgcn_readfirstlane(sp[i].op);
        const int ia = __builtin_amdgcn_readfirstlane(sp[i].a);
        const int ib = __builtin_amdgcn_readfirstlane(sp[i].b);
        const int io = __builtin_amdgcn_readfirstlane(sp[i].out);
        const double x = ia < 0 ? 0.0 : (double)sv[ia];
        const double y = ib < 0 ? 0.0 : (double)sv[ib];
        double r;
        switch (op) {
          case SI_CONST: r = sp[i].k; break;
          case SI_ADD: r = __dadd_rn(x, y); break;
          case SI_SUB: r = __dsub_rn(x, y); break;
          case SI_MUL: r = __dmul_rn(x, y); break;
          case SI_DIV: r = __ddiv_rn(x, y); break;
          case SI_MIN: r = js_min(x, y); break;
          case SI_MAX: r = js_max(x, y); break;
          case SI_ADDK: r = __dadd_rn(x, sp[i].k); break;
          case SI_MULK: r = __dmul_rn(x, sp[i].k); break;
          default: r = __dsqrt_rn(x);
        }
        if (threadIdx.x == 0) sv[io] = (float)r;
        __builtin_amdgcn_wave_barrier();
      }
    }
    __syncthreads();   // the window has run before the next one is staged
  }
  for (int i = threadIdx.x; i < a.nvals; i += kThreads) a.vals[i] = sv[i];
  if (threadIdx.x == 0) __hip_atomic_store(&a.counters[a.nslots], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

void adam_multi(const AdamChunk* chunks, int64_t nchunks, const float* lrt, AdamHyper h, const float* vals,
                hipStream_t st) {
  if (nchunks <= 0) return;
  const int64_t blocks = nchunks < 8192 ? nchunks : 8192;
  klaunch(k_opt_chunks<false>, (int)blocks, kThreads, 0, st, chunks, nchunks, lrt, h, vals);
}

void sgd_multi(const AdamChunk* chunks, int64_t nchunks, const float* lr, const float* vals, hipStream_t st) {
  if (nchunks <= 0) return;
  const int64_t blocks = nchunks < 8192 ? nchunks : 8192;
  klaunch(k_opt_chunks<true>, (int)blocks, kThreads, 0, st, chunks, nchunks, lr, AdamHyper{}, vals);
}

void grad_norms(const NormLaunch& a, hipStream_t st) {
  if (a.nchunks <= 0 || a.nchunks > 0x7fffffff) return;
  klaunch(k_grad_norms, (unsigned)a.nchunks, kThreads, 0, st, a);
}

}  // namespace tgk
