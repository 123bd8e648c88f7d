// Fused multi-tensor Adam / AdamW update for gfx950: one launch updates every parameter
// in place (p, m, v), replacing the reference's three kernels and three writeback copies
// per parameter (src/codegen.ts:841-905, src/runtime.ts:354-356).
//
// Per element, in f64 from the f32 operands, each result rounded to f32 once:
//   m' = b1*m + (1-b1)*g
//   v' = b2*v + ((1-b2)*g)*g
//   p' = shrink*p - (lrt*m') / (sqrt(v') + eps)       (m', v' as stored f32 values)
// which is the numeric convention of the CPU oracle, so updates are bit-identical to it.
// Every operation is an explicitly rounded intrinsic: no contraction into FMA.
// HBM traffic: 28 bytes per parameter (read p, g, m, v; write p, m, v).
#include "kernels.h"

namespace tgk {
namespace {

constexpr int kThreads = 256;
static_assert(kAdamChunk == kThreads * 8, "a thread updates two float4 of a full chunk");

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

// Block b updates chunks b, b + grid, ...: one descriptor load per chunk, then every
// operand of a full, 16-byte aligned chunk as two float4 per thread, all loads issued
// before the arithmetic; partial or unaligned chunks go element by element.
__global__ __launch_bounds__(kThreads) void k_adam_chunks(const AdamChunk* __restrict__ cs, int64_t nchunks,
                                                          const float* __restrict__ lrtp, AdamHyper h) {
  const double lrt = (double)*lrtp;
  for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const AdamChunk k = cs[c];
    const double shrink = k.shrink_ptr ? (double)*k.shrink_ptr : k.shrink;
    float* __restrict__ P = k.p;
    float* __restrict__ M = k.m;
    float* __restrict__ V = k.v;
    const float* __restrict__ G = k.g;
    const bool vec = k.n == kAdamChunk &&
                     ((reinterpret_cast<uintptr_t>(P) | reinterpret_cast<uintptr_t>(M) |
                       reinterpret_cast<uintptr_t>(V) | reinterpret_cast<uintptr_t>(G)) & 15) == 0;
    if (vec) {
      float4 g[2], m[2], v[2], p[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int q = threadIdx.x + u * kThreads;
        g[u] = reinterpret_cast<const float4*>(G)[q];
        m[u] = reinterpret_cast<const float4*>(M)[q];
        v[u] = reinterpret_cast<const float4*>(V)[q];
        p[u] = reinterpret_cast<const float4*>(P)[q];
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const Upd a = adam_elem(g[u].x, m[u].x, v[u].x, p[u].x, lrt, shrink, h);
        const Upd b = adam_elem(g[u].y, m[u].y, v[u].y, p[u].y, lrt, shrink, h);
        const Upd d = adam_elem(g[u].z, m[u].z, v[u].z, p[u].z, lrt, shrink, h);
        const Upd e = adam_elem(g[u].w, m[u].w, v[u].w, p[u].w, lrt, shrink, h);
        const int q = threadIdx.x + u * kThreads;
        reinterpret_cast<float4*>(P)[q] = make_float4(a.p, b.p, d.p, e.p);
        reinterpret_cast<float4*>(M)[q] = make_float4(a.m, b.m, d.m, e.m);
        reinterpret_cast<float4*>(V)[q] = make_float4(a.v, b.v, d.v, e.v);
      }
    } else {
      for (int64_t i = threadIdx.x; i < k.n; i += kThreads) {
        const Upd a = adam_elem(G[i], M[i], V[i], P[i], lrt, shrink, h);
        P[i] = a.p;
        M[i] = a.m;
        V[i] = a.v;
      }
    }
  }
}

}  // namespace

void adam_multi(const AdamChunk* chunks, int64_t nchunks, const float* lrt, AdamHyper h, hipStream_t st) {
  if (nchunks <= 0) return;
  const int64_t blocks = nchunks < 8192 ? nchunks : 8192;
  k_adam_chunks<<<(int)blocks, kThreads, 0, st>>>(chunks, nchunks, lrt, h);
}

}  // namespace tgk
