// f32 GEMM on the gfx950 matrix cores (v_mfma_f32_32x32x2_f32).
//
// C[z][m][n] = sum_k A[z][m][k] * B[z][k][n] with arbitrary element strides, so the IR's
// transposes (swapAxes before matmul, splitHeads / mergeHeads permutes) are read in place
// rather than materialised. The batch index z splits as (z / bdiv, z % bdiv) with one
// stride each, which covers [B, H, T, d] head views.
//
// Block tile BM x BN x 16 staged through LDS (k-major, padded rows: conflict-free MFMA
// operand reads), 256 threads = 4 waves in a 2 x 2 grid, each wave owning
// (BM/2) x (BN/2) built from 32 x 32 MFMA tiles. The next k-tile is prefetched into
// registers while the current one is multiplied. Tails in M, N and K are zero-filled
// on load and masked on store. Small-output / long-K problems (weight gradients) use a
// deterministic split-K: each split writes its own partial tile and a second kernel
// sums the partials in split order (no atomics).
#include "kernels.h"

namespace tgk {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 16;
constexpr int kThreads = 256;

struct GemmArgs {
  GemmDesc d;
  int64_t k_per_split;
  int splits;
  float* out;        // C, or the split-K workspace
  int64_t sOs, sOz;  // workspace strides (split, batch) when splitting
};

template <int BM, int BN>
__global__ __launch_bounds__(kThreads) void k_gemm(GemmArgs g) {
  constexpr int WM = BM / 2, WN = BN / 2;       // wave tile
  constexpr int TM = WM / 32, TN = WN / 32;     // MFMA tiles per wave
  constexpr int LDA = BM + 4, LDB = BN + 4;
  constexpr int A_PER_T = BM * kBK / kThreads;  // elements each thread stages
  constexpr int B_PER_T = BN * kBK / kThreads;
  __shared__ float As[kBK * LDA];
  __shared__ float Bs[kBK * LDB];

  const GemmDesc& d = g.d;
  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int wave = tid / 64;
  const int wm0 = (wave / 2) * WM, wn0 = (wave % 2) * WN;

  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t zz = blockIdx.z / g.splits;
  const int split = blockIdx.z % g.splits;
  const int64_t z0 = zz / d.bdiv, z1 = zz % d.bdiv;
  const float* A = d.A + z0 * d.sAz0 + z1 * d.sAz1;
  const float* B = d.B + z0 * d.sBz0 + z1 * d.sBz1;
  const int64_t kbeg = split * g.k_per_split;
  const int64_t kend = min(d.K, kbeg + g.k_per_split);

  // Thread -> staged element mapping: the unit-stride dimension varies fastest across
  // threads so global loads coalesce.
  const bool a_kfast = d.sAk == 1;
  const bool b_nfast = d.sBn == 1 || d.sBk != 1;

  float ra[A_PER_T], rb[B_PER_T];

  auto load_tiles = [&](int64_t k0) {
#pragma unroll
    for (int e = 0; e < A_PER_T; ++e) {
      int idx = tid + e * kThreads;
      int mm, kk;
      if (a_kfast) { kk = idx % kBK; mm = idx / kBK; } else { mm = idx % BM; kk = idx / BM; }
      int64_t gm = m0 + mm, gk = k0 + kk;
      ra[e] = (gm < d.M && gk < kend) ? A[gm * d.sAm + gk * d.sAk] : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < B_PER_T; ++e) {
      int idx = tid + e * kThreads;
      int nn, kk;
      if (b_nfast) { nn = idx % BN; kk = idx / BN; } else { kk = idx % kBK; nn = idx / kBK; }
      int64_t gn = n0 + nn, gk = k0 + kk;
      rb[e] = (gn < d.N && gk < kend) ? B[gk * d.sBk + gn * d.sBn] : 0.0f;
    }
  };
  auto store_tiles = [&]() {
#pragma unroll
    for (int e = 0; e < A_PER_T; ++e) {
      int idx = tid + e * kThreads;
      int mm, kk;
      if (a_kfast) { kk = idx % kBK; mm = idx / kBK; } else { mm = idx % BM; kk = idx / BM; }
      As[kk * LDA + mm] = ra[e];
    }
#pragma unroll
    for (int e = 0; e < B_PER_T; ++e) {
      int idx = tid + e * kThreads;
      int nn, kk;
      if (b_nfast) { nn = idx % BN; kk = idx / BN; } else { kk = idx % kBK; nn = idx / kBK; }
      Bs[kk * LDB + nn] = rb[e];
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int lrow = lane % 32, lk = lane / 32;
  if (kbeg < kend) load_tiles(kbeg);
  for (int64_t k0 = kbeg; k0 < kend; k0 += kBK) {
    __syncthreads();
    store_tiles();
    __syncthreads();
    if (k0 + kBK < kend) load_tiles(k0 + kBK);
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 2) {
      float av[TM], bv[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) av[i] = As[(ks + lk) * LDA + wm0 + i * 32 + lrow];
#pragma unroll
      for (int j = 0; j < TN; ++j) bv[j] = Bs[(ks + lk) * LDB + wn0 + j * 32 + lrow];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
  }

  // Store: register r of lane l holds row (r/4)*8 + (l/32)*4 + r%4, column l%32.
  float* O;
  int64_t sOm, sOn;
  if (g.splits > 1) {
    O = g.out + split * g.sOs + zz * g.sOz;
    sOm = d.N; sOn = 1;
  } else {
    O = d.C + z0 * d.sCz0 + z1 * d.sCz1;
    sOm = d.sCm; sOn = d.sCn;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t gn = n0 + wn0 + j * 32 + lrow;
      if (gn >= d.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t gm = m0 + wm0 + i * 32 + (r / 4) * 8 + lk * 4 + (r % 4);
        if (gm < d.M) O[gm * sOm + gn * sOn] = acc[i][j][r];
      }
    }
}

// Sum split-K partials in split order into C.
__global__ void k_splitk_reduce(const float* __restrict__ work, int splits, int64_t sOs, GemmDesc d) {
  const int64_t MN = d.M * d.N, total = MN * d.batch;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.0f;
    for (int sp = 0; sp < splits; ++sp) s += work[sp * sOs + i];
    const int64_t zz = i / MN, r = i % MN, m = r / d.N, n = r % d.N;
    const int64_t z0 = zz / d.bdiv, z1 = zz % d.bdiv;
    d.C[z0 * d.sCz0 + z1 * d.sCz1 + m * d.sCm + n * d.sCn] = s;
  }
}

struct Plan { int bm, bn, splits; int64_t kps; };

Plan plan_for(const GemmDesc& d) {
  auto tiles = [&](int bm, int bn) { return ((d.M + bm - 1) / bm) * ((d.N + bn - 1) / bn) * d.batch; };
  Plan p{64, 64, 1, d.K};
  if (tiles(128, 128) >= 256) p = Plan{128, 128, 1, d.K};
  else if (tiles(128, 64) >= 256) p = Plan{128, 64, 1, d.K};
  else if (tiles(64, 128) >= 256) p = Plan{64, 128, 1, d.K};
  const int64_t t = tiles(p.bm, p.bn);
  if (t < 128 && d.K >= 1024) {
    int64_t want = (256 + t - 1) / t;
    int64_t maxs = d.K / 256;
    int64_t s = want < maxs ? want : maxs;
    if (s > 64) s = 64;
    if (s > 1) {
      int64_t kps = (d.K + s - 1) / s;
      kps = (kps + kBK - 1) / kBK * kBK;
      p.splits = (int)((d.K + kps - 1) / kps);
      p.kps = kps;
    }
  }
  return p;
}

}  // namespace

int64_t gemm_workspace_floats(const GemmDesc& d) {
  Plan p = plan_for(d);
  return p.splits > 1 ? (int64_t)p.splits * d.batch * d.M * d.N : 0;
}

void gemm(const GemmDesc& d, float* work, hipStream_t st) {
  if (d.M <= 0 || d.N <= 0 || d.batch <= 0) return;
  Plan p = plan_for(d);
  GemmArgs g{d, p.kps, p.splits, nullptr, 0, 0};
  if (p.splits > 1) {
    g.out = work;
    g.sOz = d.M * d.N;
    g.sOs = d.batch * d.M * d.N;
  }
  dim3 grid((unsigned)((d.N + p.bn - 1) / p.bn), (unsigned)((d.M + p.bm - 1) / p.bm),
            (unsigned)(d.batch * p.splits));
  if (p.bm == 128 && p.bn == 128) k_gemm<128, 128><<<grid, kThreads, 0, st>>>(g);
  else if (p.bm == 128) k_gemm<128, 64><<<grid, kThreads, 0, st>>>(g);
  else if (p.bn == 128) k_gemm<64, 128><<<grid, kThreads, 0, st>>>(g);
  else k_gemm<64, 64><<<grid, kThreads, 0, st>>>(g);
  if (p.splits > 1) {
    int64_t total = d.batch * d.M * d.N;
    int64_t b = (total + 255) / 256;
    if (b > 4096) b = 4096;
    k_splitk_reduce<<<(int)b, 256, 0, st>>>(work, p.splits, g.sOs, d);
  }
}

// ---- embedding gather / segmented scatter-add ----------------------------------------

namespace {

__global__ void k_gather_rows(const int32_t* __restrict__ idx, int64_t rows, const float* __restrict__ table, int64_t V,
                              int64_t N, float* __restrict__ out) {
  const int64_t total = rows * N;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / N, c = i % N;
    const int32_t v = idx[r];
    out[i] = (v >= 0 && v < V) ? table[(int64_t)v * N + c] : 0.0f;
  }
}

// Stable counting sort of row ids by token: rows with idx == v land in
// perm[offs[v] .. offs[v+1]) in increasing row order; tokens outside [0, V) are dropped.
// One 256-thread block: integer-atomic histogram, exclusive scan, then one wavefront
// places rows 64 at a time — a lane's rank among equal tokens is counted with shuffles,
// so the order within a bucket is the row order. `cur` is V ints of scratch.
__global__ __launch_bounds__(256) void k_bucket_rows(const int32_t* __restrict__ idx, int64_t rows, int64_t V,
                                                     int32_t* __restrict__ perm, int32_t* __restrict__ offs,
                                                     int32_t* __restrict__ cur) {
  for (int64_t v = threadIdx.x; v <= V; v += blockDim.x) offs[v] = 0;
  __syncthreads();
  for (int64_t r = threadIdx.x; r < rows; r += blockDim.x) {
    int32_t t = idx[r];
    if (t >= 0 && t < V) atomicAdd(&offs[t + 1], 1);
  }
  __threadfence_block();
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int64_t v = 0; v < V; ++v) { offs[v + 1] += offs[v]; cur[v] = offs[v]; }
  }
  __threadfence_block();
  __syncthreads();
  if (threadIdx.x >= 64) return;
  const int lane = threadIdx.x;
  for (int64_t r0 = 0; r0 < rows; r0 += 64) {
    const int64_t r = r0 + lane;
    int32_t t = r < rows ? idx[r] : -1;
    if (t < 0 || t >= V) t = -1;
    int rank = 0, later = 0;
    for (int j = 0; j < 64; ++j) {
      int32_t tj = __shfl(t, j, 64);
      if (tj == t) { if (j < lane) ++rank; else if (j > lane) ++later; }
    }
    int32_t base = t >= 0 ? cur[t] : 0;
    if (t >= 0) perm[base + rank] = (int32_t)r;
    if (t >= 0 && later == 0) cur[t] = base + rank + 1;   // last lane of its token group
    __threadfence_block();
  }
}

__global__ void k_scatter_rows(const float* __restrict__ dy, int64_t V, int64_t N, const int32_t* __restrict__ perm,
                               const int32_t* __restrict__ offs, float* __restrict__ out) {
  const int64_t total = V * N;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = i / N, c = i % N;
    double s = 0.0;
    for (int32_t q = offs[v]; q < offs[v + 1]; ++q) s += (double)dy[(int64_t)perm[q] * N + c];
    out[i] = (float)s;
  }
}

inline int grid_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  return (int)(b > 2048 ? 2048 : (b < 1 ? 1 : b));
}

}  // namespace

void gather_rows(const int32_t* idx, int64_t rows, const float* table, int64_t V, int64_t N, float* out,
                 hipStream_t st) {
  if (rows * N <= 0) return;
  k_gather_rows<<<grid_for(rows * N), 256, 0, st>>>(idx, rows, table, V, N, out);
}

void scatter_rows(const int32_t* idx, int64_t rows, const float* dy, int64_t V, int64_t N, float* out, int32_t* perm,
                  int32_t* offs, hipStream_t st) {
  if (V * N <= 0) return;
  k_bucket_rows<<<1, 256, 0, st>>>(idx, rows, V, perm, offs, offs + V + 1);
  k_scatter_rows<<<grid_for(V * N), 256, 0, st>>>(dy, V, N, perm, offs, out);
}

}  // namespace tgk
