// Row reductions and softmaxes for gfx950: one 64-lane wavefront per row, lane-strided
// f64 partial sums combined with cross-lane shuffles (the reference evaluator
// accumulates these rows in f64, test/_eval.ts:206-236, 361-405). Max and argmax work on
// the exact f32 values; argmax keeps the reference's "first maximum wins, a NaN can only
// win at index 0" semantics under any combination order.
#include "kernels.h"

#include <cmath>

namespace tgk {
namespace {

constexpr int kWave = 64;
constexpr int kRowsPerBlock = 4;   // 256 threads

__device__ __forceinline__ double wave_sum(double v) {
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  for (int o = kWave / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

inline int blocks_for_rows(int64_t rows) {
  int64_t b = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  if (b > 65535 * 16) b = 65535 * 16;
  return (int)(b < 1 ? 1 : b);
}

__global__ void k_row_sum(const float* __restrict__ a, float* __restrict__ out, int64_t outer, int64_t D, double div) {
  const int lane = threadIdx.x % kWave;
  for (int64_t r = blockIdx.x * (int64_t)kRowsPerBlock + threadIdx.x / kWave; r < outer;
       r += (int64_t)gridDim.x * kRowsPerBlock) {
    const float* row = a + r * D;
    double s = 0.0;
    for (int64_t j = lane; j < D; j += kWave) s += (double)row[j];
    s = wave_sum(s);
    if (lane == 0) out[r] = (float)(s / div);
  }
}

struct ArgBest { float v; int32_t i; bool ok; };

__device__ __forceinline__ ArgBest arg_combine(ArgBest a, ArgBest b) {
  if (!b.ok) return a;
  if (!a.ok) return b;
  if (b.v > a.v) return b;
  if (a.v > b.v) return a;
  return b.i < a.i ? b : a;   // equal (or a NaN at index 0): the lower index wins
}

__global__ void k_row_argmax(const float* __restrict__ a, int32_t* __restrict__ out, int64_t outer, int64_t D) {
  const int lane = threadIdx.x % kWave;
  for (int64_t r = blockIdx.x * (int64_t)kRowsPerBlock + threadIdx.x / kWave; r < outer;
       r += (int64_t)gridDim.x * kRowsPerBlock) {
    const float* row = a + r * D;
    ArgBest best{0.0f, 0, false};
    for (int64_t j = lane; j < D; j += kWave) {
      float x = row[j];
      if (j == 0) { best = ArgBest{x, 0, true}; continue; }
      if (isnan(x)) continue;
      if (!best.ok || x > best.v) best = ArgBest{x, (int32_t)j, true};
    }
    for (int o = kWave / 2; o > 0; o >>= 1) {
      ArgBest other{__shfl_xor(best.v, o, kWave), __shfl_xor(best.i, o, kWave), (bool)__shfl_xor((int)best.ok, o, kWave)};
      best = arg_combine(best, other);
    }
    if (lane == 0) out[r] = best.i;
  }
}

__global__ void k_log_softmax(const float* __restrict__ a, float* __restrict__ out, int64_t outer, int64_t D) {
  const int lane = threadIdx.x % kWave;
  for (int64_t r = blockIdx.x * (int64_t)kRowsPerBlock + threadIdx.x / kWave; r < outer;
       r += (int64_t)gridDim.x * kRowsPerBlock) {
    const float* row = a + r * D;
    float mx = -INFINITY;
    for (int64_t j = lane; j < D; j += kWave) mx = fmaxf(mx, row[j]);
    mx = wave_max(mx);
    double s = 0.0;
    for (int64_t j = lane; j < D; j += kWave) s += exp((double)row[j] - (double)mx);
    s = wave_sum(s);
    double ls = log(s) + (double)mx;
    float* orow = out + r * D;
    for (int64_t j = lane; j < D; j += kWave) orow[j] = (float)((double)row[j] - ls);
  }
}

// Row q of each D x D matrix: softmax over columns 0..q, zeros above the diagonal.
__global__ void k_softmax_causal(const float* __restrict__ a, float* __restrict__ out, int64_t rows, int64_t D) {
  const int lane = threadIdx.x % kWave;
  for (int64_t r = blockIdx.x * (int64_t)kRowsPerBlock + threadIdx.x / kWave; r < rows;
       r += (int64_t)gridDim.x * kRowsPerBlock) {
    const int64_t q = r % D;
    const float* row = a + r * D;
    float mx = -INFINITY;
    for (int64_t j = lane; j <= q; j += kWave) mx = fmaxf(mx, row[j]);
    mx = wave_max(mx);
    double s = 0.0;
    for (int64_t j = lane; j <= q; j += kWave) s += exp((double)row[j] - (double)mx);
    s = wave_sum(s);
    float* orow = out + r * D;
    for (int64_t j = lane; j < D; j += kWave)
      orow[j] = j <= q ? (float)(exp((double)row[j] - (double)mx) / s) : 0.0f;
  }
}

__device__ __forceinline__ int64_t strided_offset(const Strided& sp, int64_t i) {
  int64_t o = 0;
  for (int d = sp.rank - 1; d >= 0; --d) {
    int64_t c = i % sp.dims[d];
    i /= sp.dims[d];
    o += c * sp.s0[d];
  }
  return o;
}

// One thread per output cell; its sources are visited in increasing flat order and
// summed in f32, as the reference evaluator does (_eval.ts:492-523).
__global__ void k_sum_to_shape(const float* __restrict__ a, float* __restrict__ out, Strided cells, Strided red,
                               int64_t ncells, int64_t nred) {
  for (int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; c < ncells; c += (int64_t)gridDim.x * blockDim.x) {
    const int64_t base = strided_offset(cells, c);
    float s = 0.0f;
    if (red.rank == 1) {
      const int64_t st = red.s0[0];
      for (int64_t r = 0; r < nred; ++r) s += a[base + r * st];
    } else {
      for (int64_t r = 0; r < nred; ++r) s += a[base + strided_offset(red, r)];
    }
    out[c] = s;
  }
}

}  // namespace

void row_sum(const float* a, float* out, int64_t outer, int64_t D, double div, hipStream_t st) {
  if (outer <= 0) return;
  k_row_sum<<<blocks_for_rows(outer), kWave * kRowsPerBlock, 0, st>>>(a, out, outer, D, div);
}

void row_argmax(const float* a, int32_t* out, int64_t outer, int64_t D, hipStream_t st) {
  if (outer <= 0) return;
  k_row_argmax<<<blocks_for_rows(outer), kWave * kRowsPerBlock, 0, st>>>(a, out, outer, D);
}

void log_softmax(const float* a, float* out, int64_t outer, int64_t D, hipStream_t st) {
  if (outer <= 0) return;
  k_log_softmax<<<blocks_for_rows(outer), kWave * kRowsPerBlock, 0, st>>>(a, out, outer, D);
}

void softmax_causal(const float* a, float* out, int64_t mats, int64_t D, hipStream_t st) {
  int64_t rows = mats * D;
  if (rows <= 0) return;
  k_softmax_causal<<<blocks_for_rows(rows), kWave * kRowsPerBlock, 0, st>>>(a, out, rows, D);
}

void sum_to_shape(const float* a, float* out, const Strided& cells, const Strided& red, int64_t ncells, int64_t nred,
                  hipStream_t st) {
  if (ncells <= 0) return;
  int64_t b = (ncells + 255) / 256;
  if (b > 4096) b = 4096;
  k_sum_to_shape<<<(int)b, 256, 0, st>>>(a, out, cells, red, ncells, nred);
}

}  // namespace tgk
