// Embedding gradient of a small vocabulary without a sort, out[v][c] = sum over rows r with
// idx[r] == v of dy[r][c]: the block body shared by the scatter launch (k_gemm.hip) and the
// column-sum launch that runs it in its first blocks beside the sums (k_reduce.hip).
#ifndef TG_SCATTER_DEV_H
#define TG_SCATTER_DEV_H
#include <hip/hip_runtime.h>
#include <cstdint>

namespace tgk {

constexpr int kScanRows = 4096;
constexpr int kScanLoads = 32;

constexpr int kScanStage = 4096;   // floats of listed rows staged at once (narrow rows)

template <int NW>
struct ScatterScanLds {
  int32_t hits[kScanRows];
  float stage[kScanStage];
  int nhit[NW];
};

// Block of NW wavefronts for token v and columns c0 .. c0 + 64 NW - 1 over rows [rb, re):
// walks idx in windows of kScanRows rows. Each wavefront ballots the rows of its share of the window whose token
// is v; the shares' counts give each wavefront its offset, so the hits land in LDS as one
// list in row order. Then every thread adds its column of the listed rows to an f64
// accumulator, in list order, kScanLoads loads in flight. The additions happen in
// increasing row order, the order of the one-hot product's k loop, whatever NW is. Returns
// the thread's column sum (f64; 0 for threads past N).
template <int NW>
__device__ __forceinline__ double scatter_scan_rows(const int32_t* __restrict__ idx, int64_t rb, int64_t rows,
                                                    const float* __restrict__ dy, int64_t N, int v, int64_t c0,
                                                    ScatterScanLds<NW>& L) {
  constexpr int Q = kScanRows / NW;   // rows per wavefront per window
  constexpr int U = kScanLoads;
  static_assert(Q % 64 == 0, "a wavefront's share of a window is whole rounds of 64 rows");
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c = c0 + threadIdx.x;
  const bool col = c < N;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  double acc = 0.0;
  for (int64_t r0 = rb; r0 < rows; r0 += kScanRows) {
    const int64_t qa = r0 + (int64_t)w * Q, qb = min(rows, qa + Q);
    int32_t t[Q / 64];
#pragma unroll
    for (int u = 0; u < Q / 64; ++u) {
      const int64_t r = qa + u * 64 + lane;
      t[u] = r < qb ? idx[r] : -1;
    }
    uint64_t m[Q / 64];
    int n = 0;
#pragma unroll
    for (int u = 0; u < Q / 64; ++u) {
      m[u] = __ballot(t[u] == v);
      n += __popcll(m[u]);
    }
    if (lane == 0) L.nhit[w] = n;
    __syncthreads();
    int base = 0, total = 0;
#pragma unroll
    for (int k = 0; k < NW; ++k) {
      const int ck = L.nhit[k];
      if (k < w) base += ck;
      total += ck;
    }
#pragma unroll
    for (int u = 0; u < Q / 64; ++u) {
      if (t[u] == v) L.hits[base + __popcll(m[u] & below)] = (int32_t)(qa + u * 64 + lane);
      base += __popcll(m[u]);
    }
    __syncthreads();
    if (c0 == 0 && N * 4 <= NW * 64) {
      // Narrow rows (N at most a quarter of the block): the whole block copies chunks of the
      // listed rows into LDS, about kScanStage / (64 NW) loads in flight per thread, then
      // each column's thread adds its column of the chunk in list order.
      const int per = kScanStage / (int)N;   // listed rows per chunk
      for (int j = 0; j < total; j += per) {
        const int cnt = min(per, total - j);
        for (int e = threadIdx.x; e < cnt * (int)N; e += NW * 64) {
          const int h = e / (int)N;
          L.stage[e] = dy[(int64_t)L.hits[j + h] * N + (e - h * (int)N)];
        }
        __syncthreads();
        if (col)
          for (int h = 0; h < cnt; ++h) acc += (double)L.stage[h * (int)N + (int)c];
        __syncthreads();
      }
    } else {
      // Every slot loads (slots past the list repeat its entry j, lanes past N read column
      // 0), so the U loads issue back to back; slots past the list add +0.0, which leaves
      // the accumulator (+0.0 or a sum that cannot be -0.0) unchanged.
      const int64_t cc = col ? c : 0;
      for (int j = 0; j < total; j += U) {
        float x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) x[u] = dy[(int64_t)L.hits[j + u < total ? j + u : j] * N + cc];
#pragma unroll
        for (int u = 0; u < U; ++u) acc += j + u < total ? (double)x[u] : 0.0;
      }
    }
    __syncthreads();   // the next window rewrites hits, nhit and stage
  }
  return acc;
}

// All rows: the column sums rounded to f32 into out[v][c].
template <int NW>
__device__ __forceinline__ void scatter_scan_block(const int32_t* __restrict__ idx, int64_t rows,
                                                   const float* __restrict__ dy, int64_t N,
                                                   float* __restrict__ out, int v, int64_t c0,
                                                   ScatterScanLds<NW>& L) {
  const double acc = scatter_scan_rows<NW>(idx, 0, rows, dy, N, v, c0, L);
  const int64_t c = c0 + threadIdx.x;
  if (c < N) out[(int64_t)v * N + c] = (float)acc;
}

}  // namespace tgk

#endif
