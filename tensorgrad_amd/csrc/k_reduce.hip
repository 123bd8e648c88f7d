// Row reductions and softmaxes for gfx950: one 64-lane wavefront per row, lane-strided
// f64 partial sums combined with cross-lane shuffles (the reference evaluator
// accumulates these rows in f64, test/_eval.ts:206-236, 361-405). Max and argmax work on
// the exact f32 values; argmax keeps the reference's "first maximum wins, a NaN can only
// win at index 0" semantics under any combination order.
#include "kernels.h"
#include "scatter_dev.h"

#include <algorithm>
#include <cmath>
#include <stdexcept>

namespace tgk {
namespace {

constexpr int kWave = 64;
constexpr int kRowsPerBlock = 4;   // 256 threads

__device__ __forceinline__ double wave_sum(double v) { return wave_allsum(v); }
__device__ __forceinline__ float wave_max(float v) { return wave_allmax(v); }

inline int blocks_for_rows(int64_t rows) {
  int64_t b = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  if (b > 65535 * 16) b = 65535 * 16;
  return (int)(b < 1 ? 1 : b);
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

// Row kernels keep a row in registers: lane l holds elements l, l + 64, ... (EPL of them,
// D <= 64 * EPL), so the row is read from memory once. EPL = 0 selects the looping form
// for long rows.
template <int EPL>
__global__ void k_log_softmax(const float* __restrict__ a, float* __restrict__ out, int64_t outer, int64_t D) {
  const int lane = threadIdx.x % kWave;
  for (int64_t r = blockIdx.x * (int64_t)kRowsPerBlock + threadIdx.x / kWave; r < outer;
       r += (int64_t)gridDim.x * kRowsPerBlock) {
    const float* row = a + r * D;
    float* orow = out + r * D;
    if (EPL > 0) {
      float x[EPL > 0 ? EPL : 1];
#pragma unroll
      for (int u = 0; u < EPL; ++u) {
        const int64_t j = lane + u * kWave;
        x[u] = j < D ? row[j] : -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int u = 0; u < EPL; ++u) mx = fmaxf(mx, x[u]);
      mx = wave_max(mx);
      double s = 0.0;
#pragma unroll
      for (int u = 0; u < EPL; ++u)
        if (lane + u * kWave < D) s += exp((double)x[u] - (double)mx);
      s = wave_sum(s);
      const double ls = log(s) + (double)mx;
#pragma unroll
      for (int u = 0; u < EPL; ++u) {
        const int64_t j = lane + u * kWave;
        if (j < D) orow[j] = (float)((double)x[u] - ls);
      }
    } else {
      float mx = -INFINITY;
      for (int64_t j = lane; j < D; j += kWave) mx = fmaxf(mx, row[j]);
      mx = wave_max(mx);
      double s = 0.0;
      for (int64_t j = lane; j < D; j += kWave) s += exp((double)row[j] - (double)mx);
      s = wave_sum(s);
      const double ls = log(s) + (double)mx;
      for (int64_t j = lane; j < D; j += kWave) orow[j] = (float)((double)row[j] - ls);
    }
  }
}

// Row q of each D x D matrix: softmax over columns 0..q, zeros above the diagonal.
template <int EPL>
__global__ void k_softmax_causal(const float* __restrict__ a, float* __restrict__ out, int64_t rows, int64_t D) {
  const int lane = threadIdx.x % kWave;
  for (int64_t r = blockIdx.x * (int64_t)kRowsPerBlock + threadIdx.x / kWave; r < rows;
       r += (int64_t)gridDim.x * kRowsPerBlock) {
    const int64_t q = r % D;
    const float* row = a + r * D;
    float* orow = out + r * D;
    if (EPL > 0) {
      float x[EPL > 0 ? EPL : 1];
#pragma unroll
      for (int u = 0; u < EPL; ++u) {
        const int64_t j = lane + u * kWave;
        x[u] = j <= q ? row[j] : -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int u = 0; u < EPL; ++u) mx = fmaxf(mx, x[u]);
      mx = wave_max(mx);
      double e[EPL > 0 ? EPL : 1];
      double s = 0.0;
#pragma unroll
      for (int u = 0; u < EPL; ++u) {
        e[u] = lane + u * kWave <= q ? exp((double)x[u] - (double)mx) : 0.0;
        if (lane + u * kWave <= q) s += e[u];
      }
      s = wave_sum(s);
#pragma unroll
      for (int u = 0; u < EPL; ++u) {
        const int64_t j = lane + u * kWave;
        if (j < D) orow[j] = j <= q ? (float)(e[u] / s) : 0.0f;
      }
    } else {
      float mx = -INFINITY;
      for (int64_t j = lane; j <= q; j += kWave) mx = fmaxf(mx, row[j]);
      mx = wave_max(mx);
      double s = 0.0;
      for (int64_t j = lane; j <= q; j += kWave) s += exp((double)row[j] - (double)mx);
      s = wave_sum(s);
      for (int64_t j = lane; j < D; j += kWave)
        orow[j] = j <= q ? (float)(exp((double)row[j] - (double)mx) / s) : 0.0f;
    }
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

// Deterministic parallel sum over a reduced index space, f64 accumulation.
// Work is split into (cell, chunk) items; each item sums a contiguous range of the
// reduced index in order, partials are combined per cell in chunk order. Two layouts:
//  * column form: the cells' last axis is unit-stride, so consecutive threads take
//    consecutive cells and every load instruction is coalesced;
//  * row form: the reduced index is innermost, so a wavefront's lanes stride over it and
//    combine through a fixed shuffle tree.
__device__ __forceinline__ int64_t red_offset(const Strided& sp, int64_t i) {
  if (sp.rank == 0) return 0;
  if (sp.rank == 1) return i * sp.s0[0];
  if (sp.rank == 2) return (i / sp.dims[1]) * sp.s0[0] + (i % sp.dims[1]) * sp.s0[1];
  return strided_offset(sp, i);
}

constexpr int kSumUnroll = 8;

// Column form: thread (cell c, chunk q) sums reduced indices [r0, r1) of cell c in order.
__global__ void k_sum_cols(const float* __restrict__ a, double* __restrict__ part, float* __restrict__ out,
                           Strided cells, Strided red, int64_t ncells, int64_t nred, int64_t chunk, int nchunks,
                           double div) {
  const int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int q = blockIdx.y;
  if (c >= ncells) return;
  const int64_t base = red_offset(cells, c);
  const int64_t r0 = q * chunk, r1 = min(nred, r0 + chunk);
  double s = 0.0;
  if (red.rank == 1) {
    const int64_t st = red.s0[0];
    const float* p = a + base + r0 * st;
    int64_t r = r0;
    // Issue kSumUnroll loads before adding them in order: keeps that many in flight.
    for (; r + kSumUnroll <= r1; r += kSumUnroll, p += kSumUnroll * st) {
      float v[kSumUnroll];
#pragma unroll
      for (int u = 0; u < kSumUnroll; ++u) v[u] = p[u * st];
#pragma unroll
      for (int u = 0; u < kSumUnroll; ++u) s += (double)v[u];
    }
    for (; r < r1; ++r, p += st) s += (double)*p;
  } else if (red.rank == 2 && r0 < r1) {
    // two reduced axes: the index split once, then stepped with a carry (no 64-bit
    // division per term); kSumUnroll loads in flight, added in index order
    const int64_t d1 = red.dims[1], s0 = red.s0[0], s1 = red.s0[1];
    int64_t hi = r0 / d1, lo = r0 - hi * d1;   // r = hi * d1 + lo
    int64_t r = r0;
    for (; r + kSumUnroll <= r1; r += kSumUnroll) {
      float v[kSumUnroll];
#pragma unroll
      for (int u = 0; u < kSumUnroll; ++u) {
        v[u] = a[base + hi * s0 + lo * s1];
        if (++lo == d1) { lo = 0; ++hi; }
      }
#pragma unroll
      for (int u = 0; u < kSumUnroll; ++u) s += (double)v[u];
    }
    for (; r < r1; ++r) {
      s += (double)a[base + hi * s0 + lo * s1];
      if (++lo == d1) { lo = 0; ++hi; }
    }
  } else if (red.rank != 2) {
    for (int64_t r = r0; r < r1; ++r) s += (double)a[base + red_offset(red, r)];
  }
  if (nchunks == 1) out[c] = (float)(s / div);
  else part[c * nchunks + q] = s;
}

// Row form: one wavefront per (cell, chunk); lane l sums indices r0 + l, r0 + l + 64, ...
// in order, then a fixed shuffle tree combines the lanes. (Finishing in each cell's last
// wavefront, as k_colsum does, measured 4-5x slower here: a hundred or more wavefronts
// per cell contend for one device-scope counter.)
__global__ void k_sum_rows(const float* __restrict__ a, double* __restrict__ part, float* __restrict__ out,
                           Strided cells, Strided red, int64_t ncells, int64_t nred, int64_t chunk, int nchunks,
                           double div) {
  const int lane = threadIdx.x % kWave;
  const int64_t items = ncells * nchunks;
  for (int64_t it = blockIdx.x * (int64_t)kRowsPerBlock + threadIdx.x / kWave; it < items;
       it += (int64_t)gridDim.x * kRowsPerBlock) {
    const int64_t c = it / nchunks;
    const int q = (int)(it % nchunks);
    const int64_t base = red_offset(cells, c);
    const int64_t r0 = q * chunk, r1 = min(nred, r0 + chunk);
    double s = 0.0;
    if (red.rank == 1) {
      const int64_t st = red.s0[0];
      const float* p = a + base;
      for (int64_t r = r0 + lane; r < r1; r += kWave * kSumUnroll) {
        float v[kSumUnroll];
#pragma unroll
        for (int u = 0; u < kSumUnroll; ++u) {   // unconditional loads (clamped): all in flight
          const int64_t j = r + u * kWave;
          v[u] = p[(j < r1 ? j : r0) * st];
        }
#pragma unroll
        for (int u = 0; u < kSumUnroll; ++u)
          if (r + u * kWave < r1) s += (double)v[u];
      }
    } else if (red.rank == 2) {
      // two reduced axes: each lane splits its first index once and steps by the
      // wavefront width with a carry (no 64-bit division per term); kSumUnroll loads in
      // flight per lane, added in index order
      const int64_t d1 = red.dims[1], s0 = red.s0[0], s1 = red.s0[1];
      if (r0 + lane < r1) {
        int64_t hi = (r0 + lane) / d1, lo = (r0 + lane) - hi * d1;   // index = hi * d1 + lo
        for (int64_t r = r0 + lane; r < r1; r += kWave * kSumUnroll) {
          // offsets first (the carry loops), then every load, then the sum: a load between
          // carry loops waited for its value before the next offset was formed
          int64_t off[kSumUnroll];
#pragma unroll
          for (int u = 0; u < kSumUnroll; ++u) {
            off[u] = r + u * kWave < r1 ? base + hi * s0 + lo * s1 : base;
            lo += kWave;
            while (lo >= d1) { lo -= d1; ++hi; }
          }
          float v[kSumUnroll];
#pragma unroll
          for (int u = 0; u < kSumUnroll; ++u) v[u] = a[off[u]];
#pragma unroll
          for (int u = 0; u < kSumUnroll; ++u)
            if (r + u * kWave < r1) s += (double)v[u];
        }
      }
    } else {
      for (int64_t r = r0 + lane; r < r1; r += kWave) s += (double)a[base + red_offset(red, r)];
    }
    s = wave_sum(s);
    if (lane == 0) {
      if (nchunks == 1) out[c] = (float)(s / div);
      else part[c * nchunks + q] = s;
    }
  }
}

// Combine the chunk partials of each cell: one wavefront per cell, lanes over chunks,
// fixed shuffle tree.
__global__ void k_sum_finish(const double* __restrict__ part, float* __restrict__ out, int64_t ncells, int nchunks,
                             double div) {
  const int lane = threadIdx.x % kWave;
  for (int64_t c = blockIdx.x * (int64_t)kRowsPerBlock + threadIdx.x / kWave; c < ncells;
       c += (int64_t)gridDim.x * kRowsPerBlock) {
    double s = 0.0;
    for (int q = lane; q < nchunks; q += kWave) s += part[c * nchunks + q];
    s = wave_sum(s);
    if (lane == 0) out[c] = (float)(s / div);
  }
}

// Column sums in one launch: out[c] = f32(sum_r x(r, c) / div), c < C, r < R, where
// x = a[r rs + c] or the f32 product a[r rs + c] * b[r rs + c], for one of several
// independent sums launched together, their blocks numbered one after another (sum i's
// from blk0; a 1-D grid with no idle blocks). A block has kColWaves wavefronts; lane l
// owns L consecutive columns (L = 4 when C allows, else 1), so block (x, y) of a sum takes
// columns [64 L x, 64 L (x + 1)) and rows [y chunk, (y + 1) chunk). Wave w sums its
// lane's columns over rows y chunk + w, + kColWaves, ... in order (f64), and the waves
// combine in order through LDS into the block's partial. The last block of a column block
// to finish (counted on counters[x]) adds the chunk partials in a fixed tree (thread j of
// a column's group takes chunks j, j + TPC, ... in order, then the group in order) and
// resets its counter, so results do not depend on scheduling and the launch leaves every
// counter at zero for the next one.
// f32(sum / div), then the mul_scalar that followed the sum in the graph (f64 product
// rounded once, as the fused groups' FO_MULS)
__device__ __forceinline__ float colsum_result(double s, const ColSum& cs) {
  const float v = (float)(s / cs.div);
  return cs.scale == 1.0 ? v : (float)((double)v * cs.scale);
}

constexpr int kColWaves = 8;
constexpr int kColThreads = kColWaves * 64;
constexpr int kColRows = 4;

// One block of a MidSum: channel c, images q chunk ... Wave w takes images b0 + w, + kColWaves,
// ...; lane l sums positions l, l + 64, ... of each (four loads in flight), all in f64 in
// that order; the wave's butterfly, then the waves in order, give the block's partial.
__device__ __forceinline__ void midsum_block(const MidSum& ms, int loc, double* wsum) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c = loc / ms.nchunks;
  const int q = loc % ms.nchunks;
  const int64_t b0 = (int64_t)q * ms.chunk, b1 = min(ms.B, b0 + ms.chunk);
  double s = 0.0;
  for (int64_t b = b0 + w; b < b1; b += kColWaves) {
    const float* row = ms.a + (b * ms.C + c) * ms.L;
    for (int64_t l = lane; l < ms.L; l += 64 * 4) {
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = l + 64 * u < ms.L ? row[l + 64 * u] : 0.0f;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (l + 64 * u < ms.L) s += (double)v[u];
    }
  }
  s = wave_allsum(s);
  if (lane == 0) wsum[w] = s;
  __syncthreads();
  if (threadIdx.x != 0) return;   // the rest is one thread's: no barrier follows
  double bs = wsum[0];
  for (int v = 1; v < kColWaves; ++v) bs += wsum[v];
  if (ms.nchunks == 1) {
    ms.out[c] = (float)bs;
    return;
  }
  // partials and the counter as device-scope atomics, as in the column sums below
  __hip_atomic_store(&ms.part[c * ms.nchunks + q], bs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  if (__hip_atomic_fetch_add(&ms.counters[c], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) !=
      (unsigned)(ms.nchunks - 1))
    return;
  double t = 0.0;
  for (int k = 0; k < ms.nchunks; ++k)
    t += __hip_atomic_load(&ms.part[c * ms.nchunks + k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  ms.out[c] = (float)t;
  __hip_atomic_store(&ms.counters[c], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// MID: the batch has [B, C, L] sums (a separate instantiation, so launches without them run
// the column-sum code alone)
template <bool MID>
__global__ __launch_bounds__(kColThreads) void k_colsum(const ColSumBatch batch) {
  if ((int)blockIdx.x < batch.sc.blocks) {   // the embedding gradient run beside the sums
    __shared__ ScatterScanLds<kColWaves> sl;
    const ColSumScatter& sc = batch.sc;
    const int vc = (int)blockIdx.x % (sc.blocks / sc.nwin), win = (int)blockIdx.x / (sc.blocks / sc.nwin);
    const int v = vc % sc.V, cy = vc / sc.V;
    const int64_t c0 = (int64_t)cy * kColThreads, c = c0 + threadIdx.x;
    const int64_t rb = (int64_t)win * sc.wrows, re = min(sc.rows, rb + sc.wrows);
    const double acc = scatter_scan_rows<kColWaves>(sc.idx, rb, re, sc.dy, sc.N, v, c0, sl);
    if (sc.nwin == 1) {
      if (c < sc.N) sc.out[(int64_t)v * sc.N + c] = (float)acc;
      return;
    }
    // partials and the counter as device-scope atomics, as in the column sums
    __shared__ int slast;
    double* part = sc.part + ((int64_t)v * sc.nwin) * sc.N;
    if (c < sc.N) __hip_atomic_store(&part[(int64_t)win * sc.N + c], acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
      slast = __hip_atomic_fetch_add(&sc.counters[vc], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              (unsigned)(sc.nwin - 1);
    __syncthreads();
    if (!slast) return;
    if (c < sc.N) {
      double t = 0.0;
      for (int k = 0; k < sc.nwin; ++k)
        t += __hip_atomic_load(&part[(int64_t)k * sc.N + c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sc.out[(int64_t)v * sc.N + c] = (float)t;
    }
    if (threadIdx.x == 0) __hip_atomic_store(&sc.counters[vc], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  int bid = (int)blockIdx.x - batch.sc.blocks;
  __shared__ double red[kColWaves][256];
  __shared__ int last;
  if (MID) {
    int mid_blocks = 0;
    for (int i = 0; i < batch.nmid; ++i) mid_blocks += (int)(batch.m[i].C * batch.m[i].nchunks);
    if (bid < mid_blocks) {   // the [B, C, L] sums' blocks
      int zm = 0;
      for (int i = 1; i < batch.nmid; ++i)
        if (bid >= batch.m[i].blk0) zm = i;
      midsum_block(batch.m[zm], bid - batch.m[zm].blk0, &red[0][0]);   // the waves' sums in red
      return;
    }
    bid -= mid_blocks;
  }
  int z = 0;
  for (int i = 1; i < batch.n; ++i)
    if (bid >= batch.s[i].blk0) z = i;
  const ColSum& cs = batch.s[z];
  const int loc = bid - cs.blk0;
  const int bx = loc % cs.nx, y = loc / cs.nx;
  constexpr int NW = kColWaves;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t C = cs.C, rs = cs.rs;
  const int nchunks = cs.nchunks;
  const int L = cs.cpl;                               // columns per lane (1 or 4)
  const int64_t c0 = ((int64_t)bx * 64 + lane) * L;   // first column of this lane
  const int64_t r0 = (int64_t)y * cs.chunk, r1 = min(cs.R, r0 + cs.chunk);
  double s[4] = {0.0, 0.0, 0.0, 0.0};
  if (c0 < C && cs.pin) {
    // f64 partial rows (a GEMM epilogue's column sums per tile row slot), added in row
    // order; eight rows' loads issued before their adds (clamped in range, masked after)
    const double* pd = cs.pin + c0;
    const int n = (int)min<int64_t>(L, C - c0);
    for (int64_t r = r0 + w; r < r1; r += 8 * NW) {
      double v[8][4];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t rr = min(r + NW * u, r1 - 1);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[u][e] = pd[rr * rs + min(e, n - 1)];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (r + NW * u < r1)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (e < n) s[e] += v[u][e];
    }
  } else if (c0 < C) {
    const float* p = cs.a + c0;
    const float* q = cs.b ? cs.b + c0 : nullptr;
    int64_t r = r0 + w;
    if (cs.aligned) {
      typedef float f4 __attribute__((ext_vector_type(4)));
      // kColRows rows in flight, added in row order; few enough registers that four
      // blocks share a CU, so a batch's blocks run in one round
      for (; r < r1; r += kColRows * NW) {
        f4 v[kColRows];
#pragma unroll
        for (int u = 0; u < kColRows; ++u)
          v[u] = r + NW * u < r1 ? *reinterpret_cast<const f4*>(p + (r + NW * u) * rs) : f4{0.f, 0.f, 0.f, 0.f};
        if (q) {
          f4 m[kColRows];
#pragma unroll
          for (int u = 0; u < kColRows; ++u)
            m[u] = r + NW * u < r1 ? *reinterpret_cast<const f4*>(q + (r + NW * u) * rs) : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int u = 0; u < kColRows; ++u) v[u] = v[u] * m[u];
        }
#pragma unroll
        for (int u = 0; u < kColRows; ++u)
          if (r + NW * u < r1)
#pragma unroll
            for (int e = 0; e < 4; ++e) s[e] += (double)v[u][e];
      }
    } else {
      const int n = (int)min<int64_t>(L, C - c0);
      for (; r < r1; r += 4 * NW) {   // four rows in flight
        float v[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) v[u][e] = e < n && r + NW * u < r1 ? p[(r + NW * u) * rs + e] : 0.0f;
        if (q) {
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              v[u][e] = v[u][e] * (e < n && r + NW * u < r1 ? q[(r + NW * u) * rs + e] : 0.0f);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (r + NW * u < r1)
#pragma unroll
            for (int e = 0; e < 4; ++e) s[e] += (double)v[u][e];
      }
    }
  }
  // the waves' sums in order, per column of the block (column lane L + e at index lane L + e)
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (e < L) red[w][lane * L + e] = s[e];
  __syncthreads();
  const int64_t cb = (int64_t)bx * 64 * L;    // first column of the block
  const int ncol = (int)min<int64_t>(64 * L, C - cb);
  // thread t < 64 L finishes column cb + t
  double bs = 0.0;
  if ((int)threadIdx.x < ncol) {
    bs = red[0][threadIdx.x];
#pragma unroll
    for (int v = 1; v < NW; ++v) bs += red[v][threadIdx.x];
  }
  if (nchunks == 1) {
    if ((int)threadIdx.x < ncol) cs.out[cb + threadIdx.x] = colsum_result(bs, cs);
    return;
  }
  // Partials, the counter and the final reads are device-scope atomic accesses: coherent
  // across the XCDs' separate L2 caches without a full L2 write-back (which a device-scope
  // fence costs). Each wave's partial stores complete (vmcnt) before the block counts in.
  double* part = cs.part;
  if ((int)threadIdx.x < ncol)
    __hip_atomic_store(&part[(int64_t)y * C + cb + threadIdx.x], bs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(&cs.counters[bx], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           (unsigned)(nchunks - 1);
  __syncthreads();
  if (!last) return;
  // The last block adds the chunks' partials: column cb + c (c < 64 L) is summed by the
  // TPC = kColThreads / (64 L) threads c + 64 L j, thread j over chunks j, j + TPC, ... in
  // order (eight loads in flight); thread c then adds the TPC sums in order j = 0, 1, ...
  const int cw = 64 * L;
  const int tpc = kColThreads / cw;
  const int col = threadIdx.x % cw, sub = threadIdx.x / cw;
  double t = 0.0;
  if (col < ncol) {
    const double* pc = part + cb + col;
    for (int ch = sub; ch < nchunks; ch += 8 * tpc) {
      double v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        v[u] = ch + u * tpc < nchunks
                   ? __hip_atomic_load(pc + (int64_t)(ch + u * tpc) * C, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                   : 0.0;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (ch + u * tpc < nchunks) t += v[u];
    }
  }
  __syncthreads();                                    // the block's reads of red are done
  reinterpret_cast<double*>(red)[threadIdx.x] = t;    // red as [tpc][64 L]
  __syncthreads();
  if ((int)threadIdx.x < ncol) {
    const double* rr = reinterpret_cast<const double*>(red);
    double u = rr[threadIdx.x];
    for (int j = 1; j < tpc; ++j) u += rr[j * cw + threadIdx.x];
    cs.out[cb + threadIdx.x] = colsum_result(u, cs);
  }
  if (threadIdx.x == 0) __hip_atomic_store(&cs.counters[bx], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Few cells with up to 64K terms each: one 256-thread block per cell. Thread t sums terms
// t, t + 256, ... in order (sixteen loads in flight), then the wavefronts' butterflies
// and the four wavefront sums in order combine them; one launch, deterministic.
__global__ __launch_bounds__(256) void k_sum_block(const float* __restrict__ a, Strided cells, Strided red,
                                                   int64_t nred, float* __restrict__ out, double div) {
  __shared__ double ws[4];
  const int64_t c = blockIdx.x;
  const int64_t base = red_offset(cells, c);
  const int64_t st = red.s0[0];
  const float* p = a + base;
  double s = 0.0;
  int64_t r = threadIdx.x;
  for (; r + 15 * 256 < nred; r += 16 * 256) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = p[(r + u * 256) * st];
#pragma unroll
    for (int u = 0; u < 16; ++u) s += (double)v[u];
  }
  for (; r < nred; r += 256) s += (double)p[r * st];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) out[c] = (float)((((ws[0] + ws[1]) + ws[2]) + ws[3]) / div);
}
bool block_form(const Strided& red, int64_t ncells, int64_t nred) {
  return red.rank == 1 && ncells <= 64 && nred <= 65536;
}

// Column-kernel shape: 64-column blocks and chunks of 64 rows (one round of sixteen loads
// in flight per lane), more rows per chunk only past 256 chunks; fewer chunks when the
// column blocks alone fill the chip.
struct ColPlan { int64_t nx; int64_t chunk; int nchunks; };
// Columns per lane of a column sum: four consecutive columns when C is a multiple of 4
// (and at least 256), so a wavefront reads 1 KiB of a row per access.
int col_lanes(int64_t C) { return C % 4 == 0 && C >= 256 ? 4 : 1; }
bool col_form(const Strided& cells, const Strided& red) {
  return cells.rank == 1 && cells.s0[0] == 1 && red.rank == 1;
}
// Row chunks sized by bytes: a block reads about 256 KiB of its sum's operands (terms = 2
// when a sum reads the product of two arrays), each of its waves between 1 and 64 rows,
// at most 256 chunks per sum. Sums of a batch then take block counts in proportion to
// their size, and the blocks of one launch finish together.
ColPlan col_plan(int64_t C, int64_t R, int terms, int scale = 1) {
  ColPlan p;
  const int L = col_lanes(C);
  p.nx = (C + 64 * L - 1) / (64 * L);
  const int64_t row_bytes = std::min<int64_t>(C, 64 * L) * 4 * std::max(terms, 1);
  int64_t rows = (262144 / row_bytes) / kColWaves * kColWaves;
  rows = std::min<int64_t>(std::max<int64_t>(rows, kColWaves), 64 * kColWaves);
  // Fewer columns than lanes (a loss mean, a small head's bias): most lanes idle, so a
  // chunk is one round of loads per wavefront and the work spreads over more blocks.
  if (C < 64) rows = kColWaves * kColRows;
  rows *= std::max(scale, 1);
  int64_t n = (R + rows - 1) / rows;
  if (n > 256) n = 256;
  if (n < 1) n = 1;
  p.chunk = (R + n - 1) / n;
  p.nchunks = (int)((R + p.chunk - 1) / p.chunk);
  if (p.nchunks < 1) p.nchunks = 1;
  return p;
}

struct SumPlan { bool cols; int64_t chunk; int nchunks; };

SumPlan sum_plan(const Strided& cells, int64_t ncells, int64_t nred) {
  SumPlan p;
  p.cols = cells.rank >= 1 && cells.s0[cells.rank - 1] == 1 && ncells >= 64;
  // Enough independent work to cover the chip's latency with kSumUnroll loads in flight
  // per lane: ~64k threads in column form (each summing >= 64 terms), ~16k wavefronts in
  // row form (each >= 512 terms); at most 256 chunks per cell.
  int64_t target = p.cols ? 65536 : 16384;
  int64_t want = (target + ncells - 1) / ncells;
  int64_t maxc = nred / (p.cols ? 64 : 512);
  if (maxc < 1) maxc = 1;
  int64_t n = want < maxc ? want : maxc;
  if (n > 256) n = 256;
  if (n < 1) n = 1;
  p.chunk = (nred + n - 1) / n;
  p.nchunks = (int)((nred + p.chunk - 1) / p.chunk);
  if (p.nchunks < 1) p.nchunks = 1;
  return p;
}

}  // namespace

void row_argmax(const float* a, int32_t* out, int64_t outer, int64_t D, hipStream_t st) {
  if (outer <= 0) return;
  klaunch(k_row_argmax, blocks_for_rows(outer), kWave * kRowsPerBlock, 0, st, a, out, outer, D);
}

#define TG_ROW_LAUNCH(KERNEL, ROWS, ...)                                                            \
  do {                                                                                              \
    const int g_ = blocks_for_rows(ROWS);                                                           \
    const int b_ = kWave * kRowsPerBlock;                                                           \
    if (D <= 64) klaunch(KERNEL<1>, g_, b_, 0, st, __VA_ARGS__);                                         \
    else if (D <= 128) klaunch(KERNEL<2>, g_, b_, 0, st, __VA_ARGS__);                                   \
    else if (D <= 256) klaunch(KERNEL<4>, g_, b_, 0, st, __VA_ARGS__);                                   \
    else if (D <= 512) klaunch(KERNEL<8>, g_, b_, 0, st, __VA_ARGS__);                                   \
    else if (D <= 1024) klaunch(KERNEL<16>, g_, b_, 0, st, __VA_ARGS__);                                 \
    else klaunch(KERNEL<0>, g_, b_, 0, st, __VA_ARGS__);                                                 \
  } while (0)

void log_softmax(const float* a, float* out, int64_t outer, int64_t D, hipStream_t st) {
  if (outer <= 0) return;
  TG_ROW_LAUNCH(k_log_softmax, outer, a, out, outer, D);
}

void softmax_causal(const float* a, float* out, int64_t mats, int64_t D, hipStream_t st) {
  int64_t rows = mats * D;
  if (rows <= 0) return;
  TG_ROW_LAUNCH(k_softmax_causal, rows, a, out, rows, D);
}

int64_t sum_workspace_doubles(const Strided& cells, const Strided& red, int64_t ncells, int64_t nred) {
  if (!col_form(cells, red) && block_form(red, ncells, nred)) return 0;
  if (col_form(cells, red)) {
    ColPlan c = col_plan(ncells, nred, 1);
    return c.nchunks > 1 ? ncells * c.nchunks : 0;
  }
  SumPlan p = sum_plan(cells, ncells, nred);
  return p.nchunks > 1 ? ncells * p.nchunks : 0;
}

ColSum colsum_desc(const float* a, const float* b, float* out, int64_t C, int64_t R, int64_t rs, double div,
                   double* part, unsigned* counters, int scale) {
  const ColPlan p = col_plan(C, R, b ? 2 : 1, scale);
  ColSum c{};
  c.a = a; c.b = b; c.out = out;
  c.C = C; c.R = R; c.rs = rs; c.chunk = p.chunk;
  c.nchunks = p.nchunks; c.nx = (int)p.nx;
  c.cpl = col_lanes(C);
  auto al = [](const float* x) { return ((uintptr_t)x & 15) == 0; };
  c.aligned = c.cpl == 4 && rs % 4 == 0 && al(a) && (!b || al(b));
  c.div = div; c.scale = 1.0; c.part = part; c.counters = counters;
  c.pin = nullptr;
  return c;
}

ColSum colsum_desc_f64(const double* pin, float* out, int64_t C, int64_t R, double* part, unsigned* counters,
                       int scale) {
  ColSum c = colsum_desc(nullptr, nullptr, out, C, R, C, 1.0, part, counters, scale);
  c.aligned = 0;
  c.pin = pin;
  return c;
}

// [B, C, L] sums: chunks of at least two images per wavefront, at most 16 per channel (the
// last block of a channel counts the arrivals on one device-scope counter)
static int64_t midsum_chunk(int64_t B) { return std::max<int64_t>(2 * kColWaves, (B + 15) / 16); }
MidSum midsum_desc(const float* a, float* out, int64_t B, int64_t C, int64_t L, double* part, unsigned* counters) {
  MidSum m{};
  m.a = a; m.out = out; m.B = B; m.C = C; m.L = L;
  m.chunk = midsum_chunk(B);
  m.nchunks = (int)((B + m.chunk - 1) / m.chunk);
  m.part = part; m.counters = counters;
  return m;
}
int64_t midsum_workspace_doubles(int64_t B, int64_t C, int64_t L) {
  (void)L;
  const int64_t ch = midsum_chunk(B), n = (B + ch - 1) / ch;
  return n > 1 ? C * n : 0;
}
int64_t midsum_counters(int64_t B, int64_t C, int64_t L) {
  (void)L;
  const int64_t ch = midsum_chunk(B);
  return (B + ch - 1) / ch > 1 ? C : 0;
}

// Row windows for the embedding gradient: about 256 blocks in all, windows of at least 512
// rows (a window's hits are found and summed with one memory latency or two).
int scatter_windows(int64_t rows, int64_t V, int64_t N) {
  if (rows <= 0 || V <= 0 || N <= 0) return 1;
  const int64_t vc = V * ((N + kColThreads - 1) / kColThreads);
  int64_t w = std::min<int64_t>((rows + 511) / 512, 256 / vc);
  if (w < 1) w = 1;
  if (w > 64) w = 64;
  const int64_t wrows = (rows + w - 1) / w;
  return (int)((rows + wrows - 1) / wrows);
}

int64_t scatter_workspace_doubles(int64_t rows, int64_t V, int64_t N) {
  const int w = scatter_windows(rows, V, N);
  return w > 1 ? V * w * N : 0;
}

int64_t scatter_counters(int64_t rows, int64_t V, int64_t N) {
  return scatter_windows(rows, V, N) > 1 ? V * ((N + kColThreads - 1) / kColThreads) : 0;
}

int64_t colsum_workspace_doubles(int64_t C, int64_t R, int terms, int scale) {
  const ColPlan p = col_plan(C, R, terms, scale);
  return p.nchunks > 1 ? C * p.nchunks : 0;
}

int64_t colsum_counters(int64_t C, int64_t R, int terms, int scale) {
  const ColPlan p = col_plan(C, R, terms, scale);
  return p.nchunks > 1 ? p.nx : 0;
}

// A batch whose column sums would take more than four blocks per CU at the default chunk
// length (C4's nine [65536, 256] bias sums: 2304 blocks) runs its chunks that many times
// longer to come to about two blocks per CU: measured on C4's batch, 121 us at 2304 blocks,
// 118 us at 1017, 96 us at 576 and 92 us at 288 (every block's LDS combine, partial store
// and arrival count is paid once per chunk). Batches within four per CU keep the default:
// C5's (about 800 blocks of [4096, C] sums) slows down with longer chunks.
int colsum_batch_scale(const int64_t* C, const int64_t* R, const int* terms, int n) {
  int64_t blocks = 0;
  for (int i = 0; i < n; ++i) {
    const ColPlan p = col_plan(C[i], R[i], terms[i]);
    blocks += p.nx * p.nchunks;
  }
  return blocks <= 1024 ? 1 : (int)((blocks + 511) / 512);
}

void colsum_batch(const ColSumBatch& b, hipStream_t st) {
  ColSumBatch bt = b;
  if (bt.n < 0) bt.n = 0;
  // the scatter's blocks first, then the sums' (numbered from 0 after them)
  bt.sc.blocks = 0;
  if (bt.sc.idx && bt.sc.V > 0 && bt.sc.N > 0) {
    const int64_t ny = (bt.sc.N + kColThreads - 1) / kColThreads;
    const int nwin = scatter_windows(bt.sc.rows, bt.sc.V, bt.sc.N);
    if ((int64_t)bt.sc.V * ny * nwin > INT32_MAX / 2) throw std::runtime_error("column sums: scatter too large");
    if (nwin > 1 && (!bt.sc.part || !bt.sc.counters)) throw std::runtime_error("column sums: scatter partials missing");
    bt.sc.nwin = nwin;
    bt.sc.wrows = (bt.sc.rows + nwin - 1) / nwin;
    bt.sc.blocks = (int)(bt.sc.V * ny * nwin);
  }
  // then the [B, C, L] sums' blocks, then the column sums' (each numbered from 0 in its range)
  if (bt.nmid < 0 || bt.nmid > kMidSumMax) throw std::runtime_error("column sums: bad [B, C, L] sum count");
  int64_t mids = 0;
  for (int i = 0; i < bt.nmid; ++i) {
    bt.m[i].blk0 = (int)mids;
    mids += bt.m[i].C * bt.m[i].nchunks;
  }
  int64_t blocks = bt.sc.blocks + mids;
  for (int i = 0; i < bt.n; ++i) {
    bt.s[i].blk0 = (int)(blocks - bt.sc.blocks - mids);
    blocks += (int64_t)bt.s[i].nx * bt.s[i].nchunks;
  }
  if (blocks <= 0) return;
  if (blocks > INT32_MAX) throw std::runtime_error("column sums: too many blocks");
  if (bt.nmid > 0) klaunch(k_colsum<true>, (unsigned)blocks, kColThreads, 0, st, bt);
  else klaunch(k_colsum<false>, (unsigned)blocks, kColThreads, 0, st, bt);
}

int64_t sum_counters(const Strided& cells, const Strided& red, int64_t ncells, int64_t nred) {
  if (col_form(cells, red)) {
    ColPlan c = col_plan(ncells, nred, 1);
    return c.nchunks > 1 ? c.nx : 0;
  }
  return 0;
}

void reduce_sum(const float* a, float* out, const Strided& cells, const Strided& red, int64_t ncells, int64_t nred,
                double div, double* work, unsigned* counters, hipStream_t st) {
  if (ncells <= 0) return;
  if (col_form(cells, red)) {
    ColSumBatch bt{};
    bt.n = 1;
    bt.s[0] = colsum_desc(a, nullptr, out, ncells, nred, red.s0[0], div, work, counters, 1);
    colsum_batch(bt, st);
    return;
  }
  if (block_form(red, ncells, nred)) {
    klaunch(k_sum_block, (unsigned)ncells, 256, 0, st, a, cells, red, nred, out, div);
    return;
  }
  SumPlan p = sum_plan(cells, ncells, nred);
  if (p.cols) {
    dim3 grid((unsigned)((ncells + 255) / 256), (unsigned)p.nchunks);
    klaunch(k_sum_cols, grid, 256, 0, st, a, work, out, cells, red, ncells, nred, p.chunk, p.nchunks, div);
  } else {
    int64_t items = ncells * p.nchunks;
    int64_t b = (items + kRowsPerBlock - 1) / kRowsPerBlock;
    if (b > 16384) b = 16384;
    klaunch(k_sum_rows, (int)b, kWave * kRowsPerBlock, 0, st, a, work, out, cells, red, ncells, nred, p.chunk, p.nchunks, div);
  }
  if (p.nchunks > 1) klaunch(k_sum_finish, blocks_for_rows(ncells), kWave * kRowsPerBlock, 0, st, work, out, ncells, p.nchunks, div);
}

}  // namespace tgk
