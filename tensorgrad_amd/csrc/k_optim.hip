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
constexpr int kPerThread = 4;
constexpr int64_t kChunk = kThreads * kPerThread;

__global__ __launch_bounds__(kThreads) void k_adam_multi(const AdamTensor* __restrict__ ts,
                                                         const int64_t* __restrict__ chunk_tensor,
                                                         const int64_t* __restrict__ chunk_start, int64_t nchunks,
                                                         const float* __restrict__ lrtp, AdamHyper h) {
  const double lrt = (double)*lrtp;
  for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const AdamTensor t = ts[chunk_tensor[c]];
    const double shrink = t.shrink_ptr ? (double)*t.shrink_ptr : t.shrink;
    const int64_t beg = chunk_start[c];
    const int64_t end = min(t.n, beg + kChunk);
    for (int64_t i = beg + threadIdx.x; i < end; i += kThreads) {
      const double g = (double)t.g[i];
      const double m = __dadd_rn(__dmul_rn(h.beta1, (double)t.m[i]), __dmul_rn(h.one_minus_beta1, g));
      const double v = __dadd_rn(__dmul_rn(h.beta2, (double)t.v[i]), __dmul_rn(__dmul_rn(h.one_minus_beta2, g), g));
      const float mf = (float)m, vf = (float)v;
      const double upd = __ddiv_rn(__dmul_rn(lrt, (double)mf), __dadd_rn(__dsqrt_rn((double)vf), h.eps));
      const double p = __dsub_rn(__dmul_rn(shrink, (double)t.p[i]), upd);
      t.m[i] = mf;
      t.v[i] = vf;
      t.p[i] = (float)p;
    }
  }
}

}  // namespace

void adam_multi(const AdamTensor* tensors, int count, const int64_t* chunk_tensor, const int64_t* chunk_start,
                int64_t nchunks, const float* lrt, AdamHyper h, hipStream_t st) {
  (void)count;
  if (nchunks <= 0) return;
  int64_t blocks = nchunks < 8192 ? nchunks : 8192;
  k_adam_multi<<<(int)blocks, kThreads, 0, st>>>(tensors, chunk_tensor, chunk_start, nchunks, lrt, h);
}

}  // namespace tgk
