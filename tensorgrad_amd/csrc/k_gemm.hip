// f32 GEMM on the gfx950 matrix cores (v_mfma_f32_32x32x2_f32).
//
// C[z][m][n] = sum_k A[z][m][k] * B[z][k][n] with arbitrary element strides, so the IR's
// transposes (swapAxes before matmul, splitHeads / mergeHeads permutes) are read in place
// rather than materialised. The batch index z splits as (z / bdiv, z % bdiv) with one
// stride each, which covers [B, H, T, d] head views.
//
// Block tile BM x BN x BK (BK = 32 for 128-row tiles, 64 for 64 x 64), 256 threads = 4
// waves in a 2 x 2 grid, each wave owning (BM/2) x (BN/2) built from 32 x 32 MFMA tiles.
//
// k-permuted operand mapping: an MFMA consumes k-pairs, lane half h supplying k index h.
// Within every group of 8 consecutive k, MFMA number j takes k = 4h + j for lane half h,
// so over j = 0..3 the two halves cover all 8 k and a lane needs 4 *consecutive* k values
// per operand. Sums over k are unchanged (every A[m][k] still meets B[k][n]).
//
// Each operand is staged in LDS in the layout it has in memory, so global loads and LDS
// writes are both 128-bit and nothing is transposed on the way in:
//  * k-contiguous operand: LDS rows [r][BK k] padded by 4 floats; a lane's 4 k values
//    are one 128-bit LDS read;
//  * row-contiguous operand: LDS rows [k][rows + 8] (the +8 puts the two lane halves on
//    disjoint banks); a lane's 4 k values are four 32-bit reads.
// Interior tiles of 16-byte aligned operands load float4; tails and other strides fall
// back to bounds-checked scalar loads (zero fill). The next k-tile is prefetched into
// registers while the current one is multiplied and then stored into the other half of
// a double-buffered LDS stage, so each stage needs a single barrier.
//
// Tiles are numbered so that each of the chip's 8 XCDs (which take workgroups round
// robin and each own an L2) receives a contiguous run of tiles, n fastest: the A rows of
// a tile row are then fetched into one L2 instead of several.
//
// Accumulation is blocked: each BK-k stage accumulates into a fresh MFMA accumulator
// that is then added to the running sum, which keeps the f32 rounding error of long
// reductions well below that of one running sum over all of K. Small-output / long-K problems (weight
// gradients) use a deterministic split-K: each split writes its own partial tile and a
// second kernel sums the partials in split order (no atomics).
#include "kernels.h"
#include "scatter_dev.h"

#include <stdexcept>
#include <cstdlib>

namespace tgk {
namespace {

using namespace gd;

constexpr int kThreads = 256;

// One operand's ROWS x BK tile: element (r, k) at X[r*sr + k*sk].
template <int ROWS, int BK, bool KFAST>
struct Tile {
  static constexpr int LD = KFAST ? BK + 4 : ROWS + 8;
  static constexpr int SIZE = KFAST ? ROWS * LD : BK * LD;
  static constexpr int Q = ROWS * BK / (4 * kThreads);
  static_assert(Q >= 1, "tile too small for the block");
  f32x4 q[Q];

  __device__ __forceinline__ static void coords(int idx, int& rr, int& kk) {
    if (KFAST) { rr = idx / (BK / 4); kk = (idx % (BK / 4)) * 4; }
    else { rr = (idx % (ROWS / 4)) * 4; kk = idx / (ROWS / 4); }
  }

  __device__ __forceinline__ void load(const float* X, int64_t sr, int64_t sk, int64_t r0, int64_t rlim, int64_t k0,
                                       int64_t klim, bool vec_ok, int tid) {
#pragma unroll
    for (int e = 0; e < Q; ++e) {
      int rr, kk;
      coords(tid + e * kThreads, rr, kk);
      const int64_t gr = r0 + rr, gk = k0 + kk;
      if (KFAST) {
        if (vec_ok && gr < rlim && gk + 3 < klim) {
          q[e] = *reinterpret_cast<const f32x4*>(X + gr * sr + gk);
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u) q[e][u] = (gr < rlim && gk + u < klim) ? X[gr * sr + (gk + u) * sk] : 0.0f;
        }
      } else {
        if (vec_ok && gr + 3 < rlim && gk < klim) {
          q[e] = *reinterpret_cast<const f32x4*>(X + gr + gk * sk);
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u) q[e][u] = (gr + u < rlim && gk < klim) ? X[(gr + u) * sr + gk * sk] : 0.0f;
        }
      }
    }
  }

  __device__ __forceinline__ void store(float* L, int tid) const {
#pragma unroll
    for (int e = 0; e < Q; ++e) {
      int rr, kk;
      coords(tid + e * kThreads, rr, kk);
      if (KFAST) *reinterpret_cast<f32x4*>(L + rr * LD + kk) = q[e];
      else *reinterpret_cast<f32x4*>(L + kk * LD + rr) = q[e];
    }
  }

  // The 4 consecutive-k values (kb .. kb+3) of row `row`.
  __device__ __forceinline__ static f32x4 frag(const float* L, int row, int kb) {
    if (KFAST) return *reinterpret_cast<const f32x4*>(L + row * LD + kb);
    f32x4 v;
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = L[(kb + u) * LD + row];
    return v;
  }
};

template <int BM, int BN, int BK, bool AK, bool BKF>
__global__ __launch_bounds__(kThreads) void k_gemm(GemmArgs g) {
  constexpr int WM = BM / 2, WN = BN / 2;       // wave tile
  constexpr int TM = WM / 32, TN = WN / 32;     // MFMA tiles per wave
  constexpr int NG = BK / 8;                    // k-groups of 8 per stage
  using TA = Tile<BM, BK, AK>;
  using TB = Tile<BN, BK, BKF>;
  // Two stages of LDS: stage s+1 is stored while stage s is multiplied, so each stage
  // needs one barrier.
  __shared__ __attribute__((aligned(16))) float As[2][TA::SIZE];
  __shared__ __attribute__((aligned(16))) float Bs[2][TB::SIZE];

  const GemmDesc& d = g.d;
  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int wave = tid / 64;
  const int wm0 = (wave / 2) * WM, wn0 = (wave % 2) * WN;

  // XCD-contiguous tile numbering (see the header comment).
  const uint32_t nblk = gridDim.x;
  uint32_t b = blockIdx.x;
  if (nblk % kXcds == 0) b = (b % kXcds) * (nblk / kXcds) + b / kXcds;
  const uint32_t tn = b % g.tiles_n;
  const uint32_t rest = b / g.tiles_n;
  const uint32_t tm = rest % g.tiles_m;
  const uint32_t zs = rest / g.tiles_m;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t zz = zs / g.splits;
  const int split = zs % g.splits;
  const int64_t z0 = zz / d.bdiv, z1 = zz % d.bdiv;
  const float* A = d.A + z0 * d.sAz0 + z1 * d.sAz1;
  const float* B = d.B + z0 * d.sBz0 + z1 * d.sBz1;
  const int64_t kbeg = split * g.k_per_split;
  const int64_t kend = min(d.K, kbeg + g.k_per_split);

  const bool a_vec = ((uintptr_t)A & 15) == 0 && (AK ? (d.sAm & 3) == 0 : (d.sAm == 1 && (d.sAk & 3) == 0));
  const bool b_vec = ((uintptr_t)B & 15) == 0 && (BKF ? (d.sBn & 3) == 0 : (d.sBn == 1 && (d.sBk & 3) == 0));

  TA sa;
  TB sb;
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int lrow = lane % 32, h = lane / 32;
  const int nst = kbeg < kend ? (int)((kend - kbeg + BK - 1) / BK) : 0;
  if (nst > 0) {
    sa.load(A, d.sAm, d.sAk, m0, d.M, kbeg, kend, a_vec, tid);
    sb.load(B, d.sBn, d.sBk, n0, d.N, kbeg, kend, b_vec, tid);
    sa.store(As[0], tid);
    sb.store(Bs[0], tid);
  }
  __syncthreads();
  for (int st = 0; st < nst; ++st) {
    const int cur = st & 1;
    const bool more = st + 1 < nst;
    if (more) {
      const int64_t k1 = kbeg + (int64_t)(st + 1) * BK;
      sa.load(A, d.sAm, d.sAk, m0, d.M, k1, kend, a_vec, tid);
      sb.load(B, d.sBn, d.sBk, n0, d.N, k1, kend, b_vec, tid);
    }
    const float* Ac = As[cur];
    const float* Bc = Bs[cur];
    // One fresh accumulator per stage (blocked summation over k, see header).
    f32x16 part[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) part[i][j][r] = 0.0f;
    f32x4 av[2][TM], bv[2][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) av[0][i] = TA::frag(Ac, wm0 + i * 32 + lrow, h * 4);
#pragma unroll
    for (int j = 0; j < TN; ++j) bv[0][j] = TB::frag(Bc, wn0 + j * 32 + lrow, h * 4);
#pragma unroll
    for (int grp = 0; grp < NG; ++grp) {
      const int c = grp & 1;
      if (grp + 1 < NG) {   // fragments of the next k-group while this one multiplies
        const int kb = (grp + 1) * 8 + h * 4;
#pragma unroll
        for (int i = 0; i < TM; ++i) av[c ^ 1][i] = TA::frag(Ac, wm0 + i * 32 + lrow, kb);
#pragma unroll
        for (int j = 0; j < TN; ++j) bv[c ^ 1][j] = TB::frag(Bc, wn0 + j * 32 + lrow, kb);
      }
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            part[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[c][i][jj], bv[c][j][jj], part[i][j], 0, 0, 0);
    }
    if (more) {
      sa.store(As[cur ^ 1], tid);
      sb.store(Bs[cur ^ 1], tid);
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] += part[i][j];
    __syncthreads();
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
        const int64_t gm = m0 + wm0 + i * 32 + (r / 4) * 8 + h * 4 + (r % 4);
        if (gm < d.M) O[gm * sOm + gn * sOn] = acc[i][j][r];
      }
    }
}

// ---- direct-to-LDS pipeline (gemm_dev.h) ----------------------------------------------

template <int BM, int BN, int BK, int NS, bool AK, bool BKF, int NT, int KG, bool BDW = false, bool ADW = false,
          bool KT = false, bool SEG = false, bool CAT = false>
__global__ __launch_bounds__(NT) void k_gemm_dma(GemmArgs g) {
  gemm_tile<BM, BN, BK, NS, AK, BKF, NT, KG, StoreC, BDW, ADW, KT, SEG, CAT>(g, xcd_order(blockIdx.x, gridDim.x),
                                                                            StoreC{});
}

// Several independent problems in one launch: problem p owns tile numbers
// [starts[p], starts[p + 1]); the table lives in device memory (uniform scalar loads).
template <int BM, int BN, int BK, int NS, bool AK, bool BKF, int NT, int KG>
__global__ __launch_bounds__(NT) void k_gemm_dma_group(const GemmArgs* __restrict__ table,
                                                       const uint32_t* __restrict__ starts, int n) {
  const uint32_t b = xcd_order(blockIdx.x, gridDim.x);
  int p = 0;
  for (int q = 1; q < n; ++q)
    if (starts[q] <= b) p = q;
  const GemmArgs g = table[p];
  gemm_tile<BM, BN, BK, NS, AK, BKF, NT, KG>(g, b - starts[p], StoreC{});
}

// Sum split-K partials in split order into C (eight partial loads in flight per thread).
__global__ void k_splitk_reduce(const float* __restrict__ work, int splits, int64_t sOs, GemmDesc d) {
  const int64_t MN = d.M * d.N, total = MN * d.batch;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.0f;
    for (int sp0 = 0; sp0 < splits; sp0 += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = sp0 + u < splits ? work[(sp0 + u) * sOs + i] : 0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (sp0 + u < splits) s += v[u];
    }
    const int64_t zz = i / MN, r = i % MN, m = r / d.N, n = r % d.N;
    const int64_t z0 = zz / d.bdiv, z1 = zz % d.bdiv;
    d.C[z0 * d.sCz0 + z1 * d.sCz1 + m * d.sCm + n * d.sCn] = s;
  }
}

struct Plan { int bm, bn, bk, splits; int64_t kps; };

constexpr int64_t kShortK = 1024;

Plan plan_for(const GemmDesc& d) {
  auto tiles = [&](int bm, int bn) { return ((d.M + bm - 1) / bm) * ((d.N + bn - 1) / bn) * d.batch; };
  // Tile shape: least padded work per CU, counted as (rounds of 256 tiles) x tile area, so
  // an M or N below the tile edge does not pay for MFMAs on padding; ties go to the larger
  // tile (more reuse per LDS byte).
  const Plan cand[4] = {{128, 128, 32, 1, d.K}, {128, 64, 32, 1, d.K}, {64, 128, 32, 1, d.K}, {64, 64, 64, 1, d.K}};
  Plan p = cand[3];
  int64_t best = -1;
  for (const Plan& c : cand) {
    const int64_t cost = (tiles(c.bm, c.bn) + 255) / 256 * c.bm * c.bn;
    if (best < 0 || cost < best) { best = cost; p = c; }
  }
  const int64_t t = tiles(p.bm, p.bn);
  // 64 x 64 tiles two or more per CU with short K: 32-k stages (64 KiB of LDS instead of
  // 128), so two blocks share a CU and one's operand loads overlap the other's MFMAs (long
  // K keeps the deeper 64-k ring).
  if (p.bm == 64 && p.bn == 64 && t >= 512 && d.K <= kShortK) p.bk = 32;
  if (t < 128 && d.K >= 1024) {
    int64_t want = (256 + t - 1) / t;
    int64_t maxs = d.K / 256;
    int64_t s = want < maxs ? want : maxs;
    if (s > 64) s = 64;
    if (s > 1) {
      int64_t kps = (d.K + s - 1) / s;
      kps = (kps + p.bk - 1) / p.bk * p.bk;
      p.splits = (int)((d.K + kps - 1) / kps);
      p.kps = kps;
    }
  }
  return p;
}

// Conditions of the direct-to-LDS kernel: whole BK stages in every split, 16-byte aligned
// operand bases for every batch entry, and per operand either k-contiguous rows with a
// stride multiple of 4, or contiguous rows (a row count multiple of 4) with a k stride
// multiple of 4.
bool dma_ok(const GemmDesc& d, const Plan& p, bool ak, bool bk) {
  if (d.K % p.bk != 0 || p.kps % p.bk != 0) return false;
  auto al = [](const float* x) { return ((uintptr_t)x & 15) == 0; };
  if (!al(d.A) || !al(d.B)) return false;
  if ((d.batch > 1) && ((d.sAz0 | d.sAz1 | d.sBz0 | d.sBz1) & 3)) return false;
  if (ak) { if (d.sAm & 3) return false; }
  else if (!(d.sAm == 1 && (d.sAk & 3) == 0 && d.M % 4 == 0)) return false;
  if (bk) { if (d.sBn & 3) return false; }
  else if (!(d.sBn == 1 && (d.sBk & 3) == 0 && d.N % 4 == 0)) return false;
  // per-lane byte offsets from the tile origin stay below 2^31
  const int64_t span = 128;   // rows (k-contiguous) or k rows (row-contiguous) of a tile, at most
  if ((ak ? d.sAm : d.sAk) * span * 4 >= (int64_t(1) << 31)) return false;
  if ((bk ? d.sBn : d.sBk) * span * 4 >= (int64_t(1) << 31)) return false;
  return true;
}

// The 64 x 64 direct-to-LDS kernel with a B operand whose rows are not 16-byte aligned
// (a 65-wide product side): B moves one 4-byte element per lane (the DTile DW mode), A as
// in dma_ok.
bool dma_bdw_ok(const GemmDesc& d, const Plan& p, bool ak, bool bk) {
  if (p.bm != 64 || p.bn != 64 || p.bk != 64) return false;
  if (d.K % p.bk != 0 || p.kps % p.bk != 0) return false;
  if (((uintptr_t)d.A & 15) != 0 || ((uintptr_t)d.B & 3) != 0) return false;
  if ((d.batch > 1) && ((d.sAz0 | d.sAz1) & 3)) return false;
  if (ak) { if (d.sAm & 3) return false; }
  else if (!(d.sAm == 1 && (d.sAk & 3) == 0 && d.M % 4 == 0)) return false;
  if (!bk && d.sBn != 1) return false;
  const int64_t span = 128;
  if ((ak ? d.sAm : d.sAk) * span * 4 >= (int64_t(1) << 31)) return false;
  if ((bk ? d.sBn : d.sBk) * span * 4 >= (int64_t(1) << 31)) return false;
  return true;
}

// TG_GEMM_GEN=0 in the environment sends these GEMMs to the register-staged kernel instead.
bool use_gen_dma() {
  static const bool on = !(std::getenv("TG_GEMM_GEN") && std::string(std::getenv("TG_GEMM_GEN")) == "0");
  return on;
}

// Any other GEMM whose operands each have a unit stride along k or along their rows: both
// operands move one 4-byte element per lane (no alignment needed) and the last stage of
// a split may be partial (K = 63, 319, ...): the direct-to-LDS pipeline with DW operands
// and the KT tail, on 128 x 128 tiles or 64 x 64 tiles with two k groups.
bool dma_gen_ok(const GemmDesc& d, bool ak, bool bk) {
  if (!ak && d.sAm != 1) return false;
  if (!bk && d.sBn != 1) return false;
  const int64_t span = 128;
  if ((ak ? d.sAm : d.sAk) * span * 4 >= (int64_t(1) << 31)) return false;
  if ((bk ? d.sBn : d.sBk) * span * 4 >= (int64_t(1) << 31)) return false;
  return true;
}

}  // namespace

namespace {

// ---- skinny products ---------------------------------------------------------------
// Products with few output columns (N <= 128 and not a multiple of 64: the 65-wide LM
// head's forward and weight gradient, 27- and 10-wide classifier heads) or a short, odd K
// (under 128, N <= 256), where the 64-wide tiles above spend most of their MFMAs on
// padding, and whose operands load coalesced in the layout below (A with unit row stride
// or 16-byte aligned k-contiguous rows, B with unit column stride). A block owns 16 rows and NT 16-wide column tiles (N padded to a multiple of 16
// only) over a k range, on v_mfma_f32_16x16x4f32. Operands go from global memory straight
// into MFMA registers, with no LDS staging and no barrier in the k loop: lane l holds
// A[m0 + l%16][k + 4(l/16) + s] and B[k + 4(l/16) + s][n0 + l%16] for s = 0..3, and MFMA s
// of a 16-k step takes k = 4g + s from lane group g. The four wavefronts take interleaved
// 16-k steps; a batch is 4 steps per wavefront (256 k per block), all of whose loads are
// issued before its MFMAs, so a block pays one memory latency per batch. Loads read
// clamped in-bounds addresses and select zero outside M, N and the k range. Each batch
// sums into a fresh accumulator that is added to the running sum; the four wavefronts'
// partial tiles are added in wavefront order through LDS. With splits > 1 each block
// covers kps of K and writes its partial tile to the workspace ([split][M][N]);
// k_splitk_reduce adds them in split order. Offsets are 32-bit (the host checks that every
// element offset fits).
// (the body: skinny_tile, gemm_dev.h)
template <int NT, bool AV>
__global__ __launch_bounds__(256) void k_gemm_skinny(const GemmArgs g) {
  skinny_tile<NT, AV>(g, StoreC{});
}

struct SkinnyPlan { int nt, nrb, ncb, splits, kps; bool av; };

bool skinny_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("TG_SKINNY");
    return !(e && e[0] == '0');
  }();
  return on;
}

// The plan depends on shapes and strides only (never on operand addresses), so the
// workspace sized at lowering matches the launch.
bool skinny_plan(const GemmDesc& d, SkinnyPlan& p) {
  if (!skinny_enabled() || d.batch != 1 || d.M <= 0 || d.N <= 0 || d.K <= 0) return false;
  const bool narrow_n = d.N <= 128 && d.N % 64 != 0;
  const bool short_k = d.K < 128 && d.K % 32 != 0 && d.N <= 256 && d.M * d.N <= (int64_t(1) << 21);
  if (!narrow_n && !short_k) return false;
  // 32-bit element offsets, non-negative strides
  const int64_t lim = int64_t(1) << 31;
  if (d.M >= lim || d.N >= lim || d.K >= lim) return false;
  if (d.sAm < 0 || d.sAk < 0 || d.sBk < 0 || d.sBn < 0) return false;
  if ((d.M - 1) * d.sAm + (d.K - 1) * d.sAk >= lim || (d.K - 1) * d.sBk + (d.N - 1) * d.sBn >= lim) return false;
  // coalesced operand loads only: the 16 lanes of a group read 16 consecutive rows of A
  // (unit row stride, or one 16-byte k quad per row) and 16 consecutive columns of B
  const bool aq = d.sAk == 1 && d.sAm % 4 == 0 && d.K % 4 == 0;
  if (!(d.sAm == 1 || aq) || d.sBn != 1) return false;
  p.av = aq;   // and a 16-byte aligned A, checked at launch
  const int64_t ct = (d.N + 15) / 16;
  p.nt = ct <= 8 ? (int)ct : 4;
  p.ncb = (int)((ct + p.nt - 1) / p.nt);
  p.nrb = (int)((d.M + 15) / 16);
  // with fewer blocks than half the CUs, split K to fill the CUs and to keep each block to
  // at most four batches (each costs a memory latency), down to one batch (256 k) per block
  const int64_t tiles = (int64_t)p.nrb * p.ncb, batch = 64 * kSkinnySteps;
  int64_t splits = 1;
  if (tiles < 128)
    splits = std::min<int64_t>((d.K + batch - 1) / batch,
                               std::max<int64_t>((256 + tiles - 1) / tiles, (d.K + 4 * batch - 1) / (4 * batch)));
  if (splits > 64) splits = 64;
  if (splits < 1) splits = 1;
  int64_t kps = (d.K + splits - 1) / splits;
  kps = (kps + 15) / 16 * 16;
  p.splits = (int)((d.K + kps - 1) / kps);
  p.kps = (int)kps;
  return true;
}

}  // namespace

bool gemm_is_tiny(const GemmDesc& d);

bool gemm_is_smallk(const GemmDesc& d);

int64_t gemm_workspace_floats(const GemmDesc& d) {
  if (!gemm_is_tiny(d) && gemm_is_smallk(d)) return 0;
  SkinnyPlan sk;
  if (!gemm_is_tiny(d) && skinny_plan(d, sk)) return sk.splits > 1 ? (int64_t)sk.splits * d.M * d.N : 0;
  Plan p = plan_for(d);
  return p.splits > 1 ? (int64_t)p.splits * d.batch * d.M * d.N : 0;
}

namespace {

// Small degenerate products (one of M, N, K is 1, up to kTinyMacs multiply-adds):
// tiny_tile (gemm_dev.h).
constexpr int64_t kTinyMacs = int64_t(1) << 21;

template <int L>
__global__ __launch_bounds__(256) void k_gemm_tiny(const GemmArgs g) {
  tiny_tile<L>(g, StoreC{});
}

// Short products (K <= kSmallK, many outputs): smallk_tile (gemm_dev.h). Longer K measured
// slower there than the tiles: the compiler keeps every unrolled LDS read in registers.
constexpr int kSmallK = 16;

template <int RM, int KB>
__global__ __launch_bounds__(256) void k_gemm_smallk(const GemmArgs g) {
  smallk_tile<RM, KB>(g, StoreC{});
}

}  // namespace

bool gemm_is_smallk(const GemmDesc& d) {
  return d.M > 0 && d.N > 0 && d.K > 0 && d.batch > 0 && d.K <= kSmallK && d.M * d.N * d.batch >= 65536;
}

// Rows per small-K block: 16 where that still gives four or more blocks per CU, else 8 or 4
static int smallk_rows(const GemmDesc& d) {
  const int64_t nbn = (d.N + 255) / 256;
  auto nblocks = [&](int rm) { return (d.M + rm - 1) / rm * nbn * d.batch; };
  return nblocks(16) >= 1024 ? 16 : nblocks(8) >= 1024 ? 8 : 4;
}

// Lanes per output of a tiny product (about K / 8 terms per lane) and its grid
static int tiny_lanes(const GemmDesc& d) {
  int L = 1;
  while (L < 64 && (int64_t)L * 8 < d.K) L *= 2;
  return L;
}
static int64_t tiny_blocks(const GemmDesc& d, int L) {
  const int64_t outs = d.M * d.N * d.batch, per = 256 / L;
  const int64_t b = (outs + per - 1) / per;
  return b < 65535 ? b : 65535;
}

bool gemm_is_tiny(const GemmDesc& d) {
  return d.M > 0 && d.N > 0 && d.K > 0 && d.batch > 0 && (d.M == 1 || d.N == 1 || d.K == 1) &&
         d.M * d.N <= kTinyMacs && d.K <= kTinyMacs && d.M * d.N * d.K * d.batch <= kTinyMacs;
}

void gemm(const GemmDesc& d, float* work, hipStream_t st) {
  if (d.M <= 0 || d.N <= 0 || d.batch <= 0) return;
  if (gemm_is_tiny(d)) {
    const int L = tiny_lanes(d);
    const dim3 grid((unsigned)tiny_blocks(d, L));
    const GemmArgs ga{d, d.K, 1, 0, 0, nullptr, 0, 0};
    switch (L) {
      case 1: klaunch(k_gemm_tiny<1>, grid, 256, 0, st, ga); return;
      case 2: klaunch(k_gemm_tiny<2>, grid, 256, 0, st, ga); return;
      case 4: klaunch(k_gemm_tiny<4>, grid, 256, 0, st, ga); return;
      case 8: klaunch(k_gemm_tiny<8>, grid, 256, 0, st, ga); return;
      case 16: klaunch(k_gemm_tiny<16>, grid, 256, 0, st, ga); return;
      case 32: klaunch(k_gemm_tiny<32>, grid, 256, 0, st, ga); return;
      default: klaunch(k_gemm_tiny<64>, grid, 256, 0, st, ga); return;
    }
  }
  if (gemm_is_smallk(d)) {
    const int nbn = (int)((d.N + 255) / 256);
    const int rm = smallk_rows(d);
    const int nbm = (int)((d.M + rm - 1) / rm);
    const int64_t blocks = (int64_t)nbn * nbm * d.batch;
    if (blocks >= (int64_t(1) << 31)) throw std::runtime_error("gemm: too many blocks");
    GemmArgs ga{d, d.K, 1, nbn, nbm, nullptr, 0, 0};
#define TG_SMALLK(RM_, KB_) klaunch(k_gemm_smallk<RM_, KB_>, (unsigned)blocks, 256, 0, st, ga)
#define TG_SMALLK_RM(RM_)                                                                  \
  if (d.K <= 8) TG_SMALLK(RM_, 8);                                                        \
  else TG_SMALLK(RM_, 16);
    if (rm == 16) { TG_SMALLK_RM(16) } else if (rm == 8) { TG_SMALLK_RM(8) } else { TG_SMALLK_RM(4) }
#undef TG_SMALLK_RM
#undef TG_SMALLK
    return;
  }
  SkinnyPlan sk;
  if (skinny_plan(d, sk)) {
    if (((uintptr_t)d.A & 15) != 0) sk.av = false;
    const GemmArgs a{d, sk.kps, sk.splits, sk.ncb, sk.nrb, work, 0, 0};
    const unsigned blocks = (unsigned)((int64_t)sk.nrb * sk.ncb * sk.splits);
#define TG_SKINNY(NT)                                                                 \
  case NT:                                                                             \
    if (sk.av) klaunch(k_gemm_skinny<NT, true>, blocks, 256, 0, st, a);                \
    else klaunch(k_gemm_skinny<NT, false>, blocks, 256, 0, st, a);                     \
    break;
    switch (sk.nt) {
      TG_SKINNY(1) TG_SKINNY(2) TG_SKINNY(3) TG_SKINNY(4) TG_SKINNY(5) TG_SKINNY(6) TG_SKINNY(7) TG_SKINNY(8)
      default: throw std::logic_error("skinny gemm: column tiles out of range");
    }
#undef TG_SKINNY
    if (sk.splits > 1) {
      const int64_t total = d.M * d.N;
      int64_t nb = (total + 255) / 256;
      if (nb > 4096) nb = 4096;
      klaunch(k_splitk_reduce, (int)nb, 256, 0, st, work, sk.splits, total, d);
    }
    return;
  }
  Plan p = plan_for(d);
  GemmArgs g{d, p.kps, p.splits, 0, 0, nullptr, 0, 0};
  if (p.splits > 1) {
    g.out = work;
    g.sOz = d.M * d.N;
    g.sOs = d.batch * d.M * d.N;
  }
  g.tiles_n = (int)((d.N + p.bn - 1) / p.bn);
  g.tiles_m = (int)((d.M + p.bm - 1) / p.bm);
  const int64_t blocks = (int64_t)g.tiles_n * g.tiles_m * d.batch * p.splits;
  if (blocks >= (int64_t(1) << 31)) throw std::runtime_error("gemm: too many tiles");
  const dim3 grid((unsigned)blocks);
  const bool ak = d.sAk == 1;
  const bool bk = d.sBk == 1 && d.sBn != 1;
  if (dma_ok(d, p, ak, bk)) {
#define TG_DMA_LAUNCH(BM_, BN_, BK_, NS_, NT_, KG_)                                                  \
  do {                                                                                             \
    if (ak && bk) klaunch(k_gemm_dma<BM_, BN_, BK_, NS_, true, true, NT_, KG_>, grid, NT_, 0, st, g);     \
    else if (ak) klaunch(k_gemm_dma<BM_, BN_, BK_, NS_, true, false, NT_, KG_>, grid, NT_, 0, st, g);     \
    else if (bk) klaunch(k_gemm_dma<BM_, BN_, BK_, NS_, false, true, NT_, KG_>, grid, NT_, 0, st, g);     \
    else klaunch(k_gemm_dma<BM_, BN_, BK_, NS_, false, false, NT_, KG_>, grid, NT_, 0, st, g);            \
  } while (0)
    // 128 x 128 tiles two or more per CU: a two-stage ring (64 KiB of LDS) so two blocks
    // share a CU and one's prologue and stores overlap the other's MFMAs; the ring depth
    // does not change the summation order
    if (p.bm == 128 && p.bn == 128 && blocks >= 512) TG_DMA_LAUNCH(128, 128, 32, 2, 512, 1);
    else if (p.bm == 128 && p.bn == 128) TG_DMA_LAUNCH(128, 128, 32, 3, 512, 1);
    else if (p.bm == 128) TG_DMA_LAUNCH(128, 64, 32, 3, 512, 1);
    else if (p.bn == 128) TG_DMA_LAUNCH(64, 128, 32, 3, 512, 1);
    else if (p.bk == 32) TG_DMA_LAUNCH(64, 64, 32, 4, 512, 2);
    else TG_DMA_LAUNCH(64, 64, 64, 4, 512, 2);
#undef TG_DMA_LAUNCH
  } else if (dma_bdw_ok(d, p, ak, bk)) {
    if (ak && bk) klaunch(k_gemm_dma<64, 64, 64, 4, true, true, 512, 2, true>, grid, 512, 0, st, g);
    else if (ak) klaunch(k_gemm_dma<64, 64, 64, 4, true, false, 512, 2, true>, grid, 512, 0, st, g);
    else if (bk) klaunch(k_gemm_dma<64, 64, 64, 4, false, true, 512, 2, true>, grid, 512, 0, st, g);
    else klaunch(k_gemm_dma<64, 64, 64, 4, false, false, 512, 2, true>, grid, 512, 0, st, g);
  } else if (use_gen_dma() && dma_gen_ok(d, ak, bk)) {
    // 128 x 128 tiles when the plan chose them, else 64 x 64 with 32-k stages (the plan's
    // k per split is a multiple of 32 either way)
    const int bt = p.bm == 128 && p.bn == 128 ? 128 : 64;
    g.tiles_n = (int)((d.N + bt - 1) / bt);
    g.tiles_m = (int)((d.M + bt - 1) / bt);
    const int64_t gb = (int64_t)g.tiles_n * g.tiles_m * d.batch * p.splits;
    if (gb >= (int64_t(1) << 31)) throw std::runtime_error("gemm: too many tiles");
    const dim3 grid((unsigned)gb);
#define TG_GEN_LAUNCH(BM_, NS_, KG_)                                                                          \
  do {                                                                                                        \
    if (ak && bk) klaunch(k_gemm_dma<BM_, BM_, 32, NS_, true, true, 512, KG_, true, true, true>, grid, 512, 0, st, g);   \
    else if (ak) klaunch(k_gemm_dma<BM_, BM_, 32, NS_, true, false, 512, KG_, true, true, true>, grid, 512, 0, st, g);   \
    else if (bk) klaunch(k_gemm_dma<BM_, BM_, 32, NS_, false, true, 512, KG_, true, true, true>, grid, 512, 0, st, g);   \
    else klaunch(k_gemm_dma<BM_, BM_, 32, NS_, false, false, 512, KG_, true, true, true>, grid, 512, 0, st, g);          \
  } while (0)
    if (bt == 128 && gb >= 512) TG_GEN_LAUNCH(128, 2, 1);   // two blocks per CU, as above
    else if (bt == 128) TG_GEN_LAUNCH(128, 3, 1);
    else TG_GEN_LAUNCH(64, 4, 2);
#undef TG_GEN_LAUNCH
  } else {
#define TG_GEMM_LAUNCH(BM_, BN_, BK_)                                                      \
  do {                                                                                     \
    if (ak && bk) klaunch(k_gemm<BM_, BN_, BK_, true, true>, grid, kThreads, 0, st, g);        \
    else if (ak) klaunch(k_gemm<BM_, BN_, BK_, true, false>, grid, kThreads, 0, st, g);        \
    else if (bk) klaunch(k_gemm<BM_, BN_, BK_, false, true>, grid, kThreads, 0, st, g);        \
    else klaunch(k_gemm<BM_, BN_, BK_, false, false>, grid, kThreads, 0, st, g);               \
  } while (0)
  if (p.bm == 128 && p.bn == 128) TG_GEMM_LAUNCH(128, 128, 32);
  else if (p.bm == 128) TG_GEMM_LAUNCH(128, 64, 32);
  else if (p.bn == 128) TG_GEMM_LAUNCH(64, 128, 32);
  else TG_GEMM_LAUNCH(64, 64, 64);
#undef TG_GEMM_LAUNCH
  }
  if (p.splits > 1) {
    int64_t total = d.batch * d.M * d.N;
    int64_t nb = (total + 255) / 256;
    if (nb > 4096) nb = 4096;
    klaunch(k_splitk_reduce, (int)nb, 256, 0, st, work, p.splits, g.sOs, d);
  }
}

// ---- products over a concatenation along k ---------------------------------------------
// A = [A0 | A1] along k: k < k0 from d.A (row stride d.sAm, 16-byte aligned rows), the rest
// from c.a1 (row stride c.lda1, any alignment). One launch of 128 x 128 tiles whose stages
// below k0 / 32 load A0 sixteen bytes per lane and whose later stages load A1 one element
// per lane, the partial last stage zeroed in LDS; B ([K, N], rows contiguous) runs straight
// through. Each output element is the same ordered sum over k as a plain GEMM over the
// materialised concatenation with 32-k stages.

bool gemm_cat_ok(const GemmDesc& d, const GemmCat& c) {
  if (d.batch != 1 || d.M <= 0 || d.N <= 0 || d.K <= 0) return false;
  if (d.sAk != 1 || (d.sAm & 3) || c.k0 < 32 || c.k0 % 32 != 0 || d.K <= c.k0 || c.lda1 < d.K - c.k0) return false;
  if (d.sBn != 1 || (d.sBk & 3) || (d.N & 3)) return false;
  if (((uintptr_t)d.A & 15) != 0 || ((uintptr_t)d.B & 15) != 0) return false;
  // per-lane byte offsets from the tile origin stay below 2^31 (128 rows / k rows a tile)
  const int64_t lim = int64_t(1) << 31;
  if (d.sAm * 128 * 4 >= lim || d.sBk * 128 * 4 >= lim || c.lda1 * 128 * 4 >= lim) return false;
  return (d.M + 127) / 128 * ((d.N + 127) / 128) < lim;
}

static GemmArgs cat_args(const GemmDesc& d, const GemmCat& c, int64_t& blocks) {
  GemmArgs g{d, d.K, 1, 0, 0, nullptr, 0, 0};
  g.tiles_n = (int)((d.N + 127) / 128);
  g.tiles_m = (int)((d.M + 127) / 128);
  g.catA = c.a1;
  g.catAm = c.lda1;
  g.cat_stages = (int)(c.k0 / 32);
  blocks = (int64_t)g.tiles_n * g.tiles_m;
  return g;
}

void gemm_cat(const GemmDesc& d, const GemmCat& c, hipStream_t st) {
  if (!gemm_cat_ok(d, c)) throw std::runtime_error("gemm_cat: unsupported operands");
  int64_t blocks = 0;
  const GemmArgs g = cat_args(d, c, blocks);
  // two or more tiles per CU: the two-stage ring (two blocks share a CU), as in gemm()
  if (blocks >= 512) klaunch(k_gemm_dma<128, 128, 32, 2, true, false, 512, 1, false, false, true, false, true>,
                             (unsigned)blocks, 512, 0, st, g);
  else klaunch(k_gemm_dma<128, 128, 32, 3, true, false, 512, 1, false, false, true, false, true>, (unsigned)blocks,
               512, 0, st, g);
}

bool gemm_cat_epi_cfg(const GemmDesc& d, const GemmCat& c, GemmEpiCfg& cfg, GemmArgs& g, int64_t& blocks) {
  if (!gemm_cat_ok(d, c)) return false;
  g = cat_args(d, c, blocks);
  cfg.bm = cfg.bn = 128;
  cfg.bk = 32;
  cfg.nt = 512;
  cfg.kg = 1;
  cfg.ak = true;
  cfg.bkf = false;
  cfg.ns = blocks >= 512 ? 2 : 3;
  cfg.cat = true;
  return true;
}

// ---- sums of products ------------------------------------------------------------------
// C = sum_s A_s B_s in one launch: the products' k ranges are stages of one GEMM whose
// stage st reads segment st / (K_s / BK) through its own bases. Every segment shares the
// strides, M and N of ds[0] and its K (a multiple of the plan's k stage); one batch and
// no split-K. The k order is segment after segment, each in the plain GEMM's order.

bool gemm_sum_ok(const GemmDesc* ds, int n) {
  if (n < 2 || n > kMaxSeg) return false;
  const GemmDesc& d0 = ds[0];
  if (d0.batch != 1 || d0.M <= 0 || d0.N <= 0 || d0.K <= 0) return false;
  for (int s = 1; s < n; ++s) {
    const GemmDesc& d = ds[s];
    if (d.batch != 1 || d.M != d0.M || d.N != d0.N || d.K != d0.K || d.sAm != d0.sAm || d.sAk != d0.sAk ||
        d.sBk != d0.sBk || d.sBn != d0.sBn)
      return false;
  }
  GemmDesc all = d0;
  all.K = d0.K * n;
  const Plan p = plan_for(all);
  if (p.splits != 1 || p.bk != 32 && p.bk != 64 || d0.K % p.bk != 0) return false;
  if (!(p.bm == 64 && p.bn == 64) && !(p.bm == 128 && p.bn == 128)) return false;
  const bool ak = d0.sAk == 1;
  const bool bk = d0.sBk == 1 && d0.sBn != 1;
  for (int s = 0; s < n; ++s)
    if (!dma_ok(ds[s], Plan{p.bm, p.bn, p.bk, 1, ds[s].K}, ak, bk)) return false;
  return true;
}

void gemm_sum(const GemmDesc* ds, int n, hipStream_t st) {
  if (!gemm_sum_ok(ds, n)) throw std::runtime_error("gemm_sum: unsupported operands");
  GemmDesc all = ds[0];
  all.K = ds[0].K * n;
  const Plan p = plan_for(all);
  GemmArgs g{all, all.K, 1, 0, 0, nullptr, 0, 0};
  g.tiles_n = (int)((all.N + p.bn - 1) / p.bn);
  g.tiles_m = (int)((all.M + p.bm - 1) / p.bm);
  g.nseg = n;
  g.seg_stages = (int)(ds[0].K / p.bk);
  for (int s = 0; s < n; ++s) { g.segA[s] = ds[s].A; g.segB[s] = ds[s].B; }
  const int64_t blocks = (int64_t)g.tiles_n * g.tiles_m;
  const dim3 grid((unsigned)blocks);
  const bool ak = all.sAk == 1;
  const bool bk = all.sBk == 1 && all.sBn != 1;
#define TG_SEG_LAUNCH(BM_, BK_, NS_, KG_)                                                                          \
  do {                                                                                                           \
    if (ak && bk) klaunch(k_gemm_dma<BM_, BM_, BK_, NS_, true, true, 512, KG_, false, false, false, true>, grid, 512, 0, st, g); \
    else if (ak) klaunch(k_gemm_dma<BM_, BM_, BK_, NS_, true, false, 512, KG_, false, false, false, true>, grid, 512, 0, st, g); \
    else if (bk) klaunch(k_gemm_dma<BM_, BM_, BK_, NS_, false, true, 512, KG_, false, false, false, true>, grid, 512, 0, st, g); \
    else klaunch(k_gemm_dma<BM_, BM_, BK_, NS_, false, false, 512, KG_, false, false, false, true>, grid, 512, 0, st, g);        \
  } while (0)
  if (p.bm == 128) TG_SEG_LAUNCH(128, 32, 3, 1);
  else if (p.bk == 32) TG_SEG_LAUNCH(64, 32, 4, 2);
  else TG_SEG_LAUNCH(64, 64, 4, 2);
#undef TG_SEG_LAUNCH
}

// ---- grouped GEMMs ---------------------------------------------------------------------
// Problems of one group launch run whole-K 64 x 64 tiles (two k groups of four wavefronts),
// so weight gradients with few output tiles fill the chip together instead of each
// splitting K.

int gemm_group_kind(const GemmDesc& d) {
  if (d.M <= 0 || d.N <= 0 || d.batch <= 0 || d.K <= 0) return -1;
  const Plan p{64, 64, 64, 1, d.K};
  const bool ak = d.sAk == 1;
  const bool bk = d.sBk == 1 && d.sBn != 1;
  if (!dma_ok(d, p, ak, bk)) return -1;
  return (ak ? 2 : 0) + (bk ? 1 : 0);
}

bool gemm_prefers_group(const GemmDesc& d) {
  if (gemm_group_kind(d) < 0) return false;
  const Plan p = plan_for(d);
  return p.bm == 64 && p.bn == 64 && p.splits == 1;
}

bool gemm_epi_cfg(const GemmDesc& d, GemmEpiCfg& c, GemmArgs& g, int64_t& blocks) {
  if (d.M <= 0 || d.N <= 0 || d.batch <= 0) return false;
  if (gemm_is_tiny(d)) {   // the tiny kernel gemm() runs, one batch
    if (d.batch != 1) return false;
    g = GemmArgs{d, d.K, 1, 0, 0, nullptr, 0, 0};
    c.tiny = true;
    c.bm = tiny_lanes(d);
    c.bn = c.bk = 1;
    c.nt = 256;
    c.kg = 1;
    c.ns = 0;
    c.ak = d.sAk == 1;
    c.bkf = d.sBk == 1 && d.sBn != 1;
    blocks = tiny_blocks(d, c.bm);
    return true;
  }
  {   // the skinny kernel gemm() runs (one split, one batch)
    SkinnyPlan sk;
    if (skinny_plan(d, sk)) {
      if (sk.splits != 1 || d.batch != 1) return false;
      if (((uintptr_t)d.A & 15) != 0) sk.av = false;
      g = GemmArgs{d, sk.kps, 1, sk.ncb, sk.nrb, nullptr, 0, 0};
      blocks = (int64_t)sk.nrb * sk.ncb;
      c.skinny = true;
      c.bm = sk.nt;     // column tiles per block
      c.bk = sk.av ? 1 : 0;
      c.bn = 16;
      c.nt = 256;
      c.kg = 1;
      c.ns = 0;
      c.ak = d.sAk == 1;
      c.bkf = d.sBk == 1 && d.sBn != 1;
      return true;
    }
  }
  if (gemm_is_smallk(d)) {   // the small-K kernel gemm() runs, one batch
    if (d.batch != 1) return false;
    const int rm = smallk_rows(d);
    g = GemmArgs{d, d.K, 1, (int)((d.N + 255) / 256), (int)((d.M + rm - 1) / rm), nullptr, 0, 0};
    blocks = (int64_t)g.tiles_n * g.tiles_m;
    c.smallk = true;
    c.bm = rm;
    c.bk = d.K <= 8 ? 8 : 16;
    c.bn = 256;
    c.nt = 256;
    c.kg = 1;
    c.ns = 0;
    c.ak = d.sAk == 1;
    c.bkf = d.sBk == 1 && d.sBn != 1;
    return blocks < (int64_t(1) << 31);
  }
  const Plan p = plan_for(d);
  const bool ak = d.sAk == 1;
  const bool bk = d.sBk == 1 && d.sBn != 1;
  if (p.splits != 1) return false;
  SkinnyPlan sk;
  if (!dma_ok(d, p, ak, bk) && !dma_bdw_ok(d, p, ak, bk) && use_gen_dma() && dma_gen_ok(d, ak, bk) &&
      !skinny_plan(d, sk)) {
    // the element-wise tile gemm() launches for unaligned operands / partial k stages
    const int bt = p.bm == 128 && p.bn == 128 ? 128 : 64;
    g = GemmArgs{d, p.kps, 1, 0, 0, nullptr, 0, 0};
    g.tiles_n = (int)((d.N + bt - 1) / bt);
    g.tiles_m = (int)((d.M + bt - 1) / bt);
    blocks = (int64_t)g.tiles_n * g.tiles_m * d.batch;
    c.bm = c.bn = bt;
    c.bk = 32;
    c.nt = 512;
    c.kg = bt == 128 ? 1 : 2;
    c.ns = bt == 128 ? (blocks >= 512 ? 2 : 3) : 4;
    c.ak = ak; c.bkf = bk;
    c.gen = true;
    return blocks < (int64_t(1) << 31);
  }
  if (!dma_ok(d, p, ak, bk)) return false;
  // the same instantiation gemm() launches for this plan
  c.bm = p.bm; c.bn = p.bn; c.bk = p.bk;
  c.nt = 512;
  c.kg = p.bm == 64 && p.bn == 64 ? 2 : 1;
  c.ak = ak; c.bkf = bk;
  g = GemmArgs{d, p.kps, 1, 0, 0, nullptr, 0, 0};
  g.tiles_n = (int)((d.N + p.bn - 1) / p.bn);
  g.tiles_m = (int)((d.M + p.bm - 1) / p.bm);
  blocks = (int64_t)g.tiles_n * g.tiles_m * d.batch;
  // (64 x 64 with p.bk = 32: the 64 KiB variant; 128 x 128 two or more per CU: two stages)
  c.ns = p.bm == 64 && p.bn == 64 ? 4 : (p.bm == 128 && p.bn == 128 && blocks >= 512 ? 2 : 3);
  return blocks < (int64_t(1) << 31);
}

int64_t gemm_epi_colsum_rows(const GemmEpiCfg& c, const GemmArgs& g) {
  if (c.smallk) return g.tiles_m;   // one row per block of rows
  // gemm_tile's wavefront grid: NW wavefronts per k group, 4 x 2 for eight with a 64-wide
  // tile, else 2 along M
  const int nw = c.nt / c.kg / 64;
  const int wgm = nw == 8 && c.bn == 64 ? 4 : 2;
  return (int64_t)g.tiles_m * wgm;
}

size_t gemm_group_table(const GemmDesc* ds, int n, std::vector<unsigned char>& image, int64_t& blocks, int& tiling) {
  const size_t args_bytes = (size_t)n * sizeof(GemmArgs);
  const size_t starts_off = (args_bytes + 15) / 16 * 16;
  image.assign(starts_off + (size_t)(n + 1) * sizeof(uint32_t), 0);
  GemmArgs* args = reinterpret_cast<GemmArgs*>(image.data());
  uint32_t* starts = reinterpret_cast<uint32_t*>(image.data() + starts_off);
  int64_t t = 0;
  for (int q = 0; q < n; ++q) {
    const GemmDesc& d = ds[q];
    GemmArgs g{d, d.K, 1, 0, 0, nullptr, 0, 0};
    g.tiles_n = (int)((d.N + 63) / 64);
    g.tiles_m = (int)((d.M + 63) / 64);
    args[q] = g;
    starts[q] = (uint32_t)t;
    t += (int64_t)g.tiles_n * g.tiles_m * d.batch;
  }
  starts[n] = (uint32_t)t;
  if (t >= (int64_t(1) << 31)) throw std::runtime_error("gemm group: too many tiles");
  blocks = t;
  // Two or more tiles per CU: 32-k stages. With every K short, the plain launch's 64 KiB
  // variant (two blocks per CU). With a long K, four wavefronts per tile and a 48 KiB
  // three-stage ring, so three blocks share a CU and overlap one another's first loads and
  // stores: at 768 tiles of K = 4096, 80 % of the f32 MFMA peak against 76 % for the 128 KiB
  // eight-wavefront tile, which runs one block per CU and its tiles one after another.
  int64_t kmax = 0;
  for (int q = 0; q < n; ++q) kmax = std::max(kmax, ds[q].K);
  tiling = t >= 512 ? (kmax <= kShortK ? 1 : 2) : 0;
  return starts_off;
}

void gemm_group(const void* dev_image, size_t starts_off, int n, int64_t blocks, int kind, int tiling,
                hipStream_t st) {
  if (n <= 0 || blocks <= 0) return;
  const GemmArgs* table = reinterpret_cast<const GemmArgs*>(dev_image);
  const uint32_t* starts = reinterpret_cast<const uint32_t*>(reinterpret_cast<const unsigned char*>(dev_image) + starts_off);
  const dim3 grid((unsigned)blocks);
  if (tiling == 2) {   // 32-k stages on four wavefronts, 48 KiB: three blocks per CU
    switch (kind) {
      case 3: klaunch(k_gemm_dma_group<64, 64, 32, 3, true, true, 256, 1>, grid, 256, 0, st, table, starts, n); return;
      case 2: klaunch(k_gemm_dma_group<64, 64, 32, 3, true, false, 256, 1>, grid, 256, 0, st, table, starts, n); return;
      case 1: klaunch(k_gemm_dma_group<64, 64, 32, 3, false, true, 256, 1>, grid, 256, 0, st, table, starts, n); return;
      case 0: klaunch(k_gemm_dma_group<64, 64, 32, 3, false, false, 256, 1>, grid, 256, 0, st, table, starts, n); return;
      default: throw std::runtime_error("gemm group: bad kind");
    }
  }
  if (tiling == 1) {   // 32-k stages: the 64 KiB-LDS variant, two blocks per CU
    switch (kind) {
      case 3: klaunch(k_gemm_dma_group<64, 64, 32, 4, true, true, 512, 2>, grid, 512, 0, st, table, starts, n); return;
      case 2: klaunch(k_gemm_dma_group<64, 64, 32, 4, true, false, 512, 2>, grid, 512, 0, st, table, starts, n); return;
      case 1: klaunch(k_gemm_dma_group<64, 64, 32, 4, false, true, 512, 2>, grid, 512, 0, st, table, starts, n); return;
      case 0: klaunch(k_gemm_dma_group<64, 64, 32, 4, false, false, 512, 2>, grid, 512, 0, st, table, starts, n); return;
      default: throw std::runtime_error("gemm group: bad kind");
    }
  }
  switch (kind) {
    case 3: klaunch(k_gemm_dma_group<64, 64, 64, 4, true, true, 512, 2>, grid, 512, 0, st, table, starts, n); break;
    case 2: klaunch(k_gemm_dma_group<64, 64, 64, 4, true, false, 512, 2>, grid, 512, 0, st, table, starts, n); break;
    case 1: klaunch(k_gemm_dma_group<64, 64, 64, 4, false, true, 512, 2>, grid, 512, 0, st, table, starts, n); break;
    case 0: klaunch(k_gemm_dma_group<64, 64, 64, 4, false, false, 512, 2>, grid, 512, 0, st, table, starts, n); break;
    default: throw std::runtime_error("gemm group: bad kind");
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

// Rows of 4k floats, 16-byte aligned: one float4 per thread, 32-bit index math.
__global__ void k_gather_rows4(const int32_t* __restrict__ idx, uint32_t rows, const float4* __restrict__ table,
                               uint32_t V, uint32_t n4, float4* __restrict__ out) {
  const uint32_t total = rows * n4;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    const uint32_t r = i / n4, c = i - r * n4;
    const int32_t v = idx[r];
    out[i] = (v >= 0 && (uint32_t)v < V) ? table[(size_t)v * n4 + c] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// Stable counting sort of row ids by token, in one block of kBucketWaves wavefronts: rows
// with idx == v land in perm[offs[v] .. offs[v+1]) in increasing row order; tokens outside
// [0, V) are dropped. Wave w of the block owns a contiguous 1 / kBucketWaves of the rows
// (all rows when V > kWaveHistV): a per-wave LDS histogram, one block-wide scan that
// yields each wave's starting cursor per token, then each wave places its rows 64 at a
// time. A lane's rank among equal tokens of its group comes from matching the token's bits
// with ballots. The scan also lays out the segment-sum work: bucket v is cut into
// ceil(count / kSeg) items starting at item cstart[v]; item i covers perm positions
// [item_rng[2i], item_rng[2i + 1]).
constexpr int kMaxBucketV = 8192;
constexpr int kWaveHistV = 1024;
constexpr int kBucketWaves = 16;   // wavefronts of the sorting block (1024 threads)
constexpr int kSeg = 16;
// s_waitcnt operand for lgkmcnt(0) alone: vmcnt 63 (bits 3:0 and 15:14), expcnt 7 (6:4),
// lgkmcnt 0 (11:8).
constexpr int kWaitLds = 0xF | (0x3 << 14) | (0x7 << 4);

__device__ __forceinline__ int block_exclusive_scan(int x, int* lds_tot, int& total) {
  // kBucketWaves wavefronts: shuffle-up scan inside each wavefront, then wavefront totals.
  const int lane = threadIdx.x % 64, w = threadIdx.x / 64;
  int inc = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(inc, o, 64);
    if (lane >= o) inc += y;
  }
  if (lane == 63) lds_tot[w] = inc;
  __syncthreads();
  int before = 0;
  total = 0;
#pragma unroll
  for (int k = 0; k < kBucketWaves; ++k) {
    const int t = lds_tot[k];
    if (k < w) before += t;
    total += t;
  }
  __syncthreads();
  return before + inc - x;
}

__global__ __launch_bounds__(kBucketWaves * 64) void k_bucket_rows(const int32_t* __restrict__ idx, int64_t rows, int64_t V,
                                                     int stash, int32_t* __restrict__ perm, int32_t* __restrict__ offs,
                                                     int32_t* __restrict__ cstart, int32_t* __restrict__ item_rng) {
  extern __shared__ int32_t lds[];
  __shared__ int tot[kBucketWaves];
  const int nw = V <= kWaveHistV ? kBucketWaves : 1;
  const int VP = (int)V + 1;            // slot V counts dropped tokens
  int32_t* cnt = lds;                   // [nw][VP]
  int32_t* tok = lds + nw * VP;         // [rows] when stash != 0
  const int lane = threadIdx.x % 64, w = threadIdx.x / 64;
  for (int i = threadIdx.x; i < nw * VP; i += blockDim.x) cnt[i] = 0;
  __syncthreads();
  const int64_t per = ((rows + nw - 1) / nw + 63) / 64 * 64;
  if (w < nw) {
    const int64_t r0 = w * per, r1 = min(rows, r0 + per);
    // Eight token loads in flight per lane before the histogram updates.
    for (int64_t rb = r0; rb < r1; rb += 64 * 8) {
      int32_t t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t r = rb + u * 64 + lane;
        t[u] = r < r1 ? idx[r] : -1;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t r = rb + u * 64 + lane;
        if (r < r1) {
          const int32_t tt = (t[u] < 0 || t[u] >= V) ? (int32_t)V : t[u];
          atomicAdd(&cnt[w * VP + tt], 1);
          if (stash) tok[r] = tt;
        }
      }
    }
  }
  __syncthreads();
  // Scan over tokens: thread j owns tokens [j*seg, (j+1)*seg).
  const int seg = (VP + kBucketWaves * 64 - 1) / (kBucketWaves * 64);
  const int v0 = threadIdx.x * seg, v1 = min(VP - 1, v0 + seg);   // token V (dropped) excluded
  int my = 0, myc = 0;
  for (int v = v0; v < v1; ++v) {
    int c = 0;
    for (int k = 0; k < nw; ++k) c += cnt[k * VP + v];
    my += c;
    myc += (c + kSeg - 1) / kSeg;
  }
  int total, totc;
  int run = block_exclusive_scan(my, tot, total);
  int runc = block_exclusive_scan(myc, tot, totc);
  for (int v = v0; v < v1; ++v) {
    int c = 0;
    offs[v] = run;
    cstart[v] = runc;
    for (int k = 0; k < nw; ++k) {
      const int ck = cnt[k * VP + v];
      cnt[k * VP + v] = run + c;        // wave k's first slot for token v
      c += ck;
    }
    const int nc = (c + kSeg - 1) / kSeg;
    for (int i = 0; i < nc; ++i) {
      item_rng[2 * (runc + i)] = run + i * kSeg;
      item_rng[2 * (runc + i) + 1] = min(run + c, run + (i + 1) * kSeg);
    }
    run += c;
    runc += nc;
  }
  if (threadIdx.x == 0) { offs[V] = total; cstart[V] = totc; }
  __syncthreads();
  if (w >= nw) return;
  int nbits = 1;
  while ((1 << nbits) < VP) ++nbits;
  const int64_t r0 = w * per, r1 = min(rows, r0 + per);
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int64_t rb = r0; rb < r1; rb += 64) {
    const int64_t r = rb + lane;
    const bool live = r < r1;
    int32_t t = (int32_t)V;
    if (live) {
      t = stash ? tok[r] : idx[r];
      if (t < 0 || t >= V) t = (int32_t)V;
    }
    uint64_t same = __ballot(live);
    for (int b = 0; b < nbits; ++b) {
      const uint64_t ones = __ballot(live && ((t >> b) & 1));
      same &= ((t >> b) & 1) ? ones : ~ones;
    }
    const int rank = __popcll(same & below);
    const int count = __popcll(same);
    const bool place = live && t < V;
    // Every lane's read of its token's cursor completes before the group's last lane
    // advances it, and the advance before the next group's reads. The waits cover LDS
    // only (lgkmcnt 0, vmcnt and expcnt left at their maximum): the perm stores stay in
    // flight across iterations.
    const int base = place ? cnt[w * VP + t] : 0;
    __builtin_amdgcn_s_waitcnt(kWaitLds);
    __builtin_amdgcn_wave_barrier();
    if (place) perm[base + rank] = (int32_t)r;
    if (place && rank == count - 1) cnt[w * VP + t] = base + count;
    __builtin_amdgcn_s_waitcnt(kWaitLds);
    __builtin_amdgcn_wave_barrier();
  }
}

// Block i sums item i — up to kSeg consecutive rows of one bucket — per column, in row
// order, in f64. The item's range and the item count load together, then the row ids,
// then the rows.
__global__ __launch_bounds__(256) void k_segment_partials(const float* __restrict__ dy, int64_t N, int64_t V,
                                                          const int32_t* __restrict__ perm,
                                                          const int32_t* __restrict__ cstart,
                                                          const int32_t* __restrict__ item_rng,
                                                          double* __restrict__ part) {
  const int i = blockIdx.x;
  const int nitems = cstart[V];
  const int j0 = item_rng[2 * i], j1 = item_rng[2 * i + 1];
  if (i >= nitems) return;
  int64_t rr[kSeg];
#pragma unroll
  for (int u = 0; u < kSeg; ++u) rr[u] = j0 + u < j1 ? (int64_t)perm[j0 + u] * N : 0;
  for (int64_t c = blockIdx.y * (int64_t)blockDim.x + threadIdx.x; c < N; c += (int64_t)gridDim.y * blockDim.x) {
    float x[kSeg];
#pragma unroll
    for (int u = 0; u < kSeg; ++u) x[u] = j0 + u < j1 ? dy[rr[u] + c] : 0.0f;
    double s = 0.0;
#pragma unroll
    for (int u = 0; u < kSeg; ++u)
      if (j0 + u < j1) s += (double)x[u];
    part[(int64_t)i * N + c] = s;
  }
}

// out[v, c] = sum of bucket v's item partials, in item (= row) order.
__global__ void k_segment_finish(const double* __restrict__ part, int64_t N, int64_t V,
                                 const int32_t* __restrict__ cstart, float* __restrict__ out) {
  const int64_t total = V * N;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = e / N, c = e % N;
    double s = 0.0;
    for (int i = cstart[v]; i < cstart[v + 1]; ++i) s += part[(int64_t)i * N + c];
    out[e] = (float)s;
  }
}

// Small vocabularies (V * rows <= kScatterScanMax) need no sort: block (v, column chunk)
// of four wavefronts runs scatter_scan_block (scatter_dev.h). One launch, no workspace.
constexpr int64_t kScatterScanMax = int64_t(1) << 22;

__global__ __launch_bounds__(256) void k_scatter_scan(const int32_t* __restrict__ idx, int64_t rows,
                                                      const float* __restrict__ dy, int64_t N,
                                                      float* __restrict__ out) {
  __shared__ ScatterScanLds<4> L;
  scatter_scan_block<4>(idx, rows, dy, N, out, (int)blockIdx.x, blockIdx.y * 256ll, L);
}

inline bool scatter_scans(int64_t rows, int64_t V) { return V * rows <= kScatterScanMax; }

inline int grid_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  return (int)(b > 2048 ? 2048 : (b < 1 ? 1 : b));
}

}  // namespace

void gather_rows(const int32_t* idx, int64_t rows, const float* table, int64_t V, int64_t N, float* out,
                 hipStream_t st) {
  if (rows * N <= 0) return;
  if (N % 4 == 0 && rows * N < (int64_t(1) << 32) && V < (int64_t(1) << 32) && ((uintptr_t)table & 15) == 0 &&
      ((uintptr_t)out & 15) == 0) {
    klaunch(k_gather_rows4, grid_for(rows * N / 4), 256, 0, st, idx, (uint32_t)rows, (const float4*)table,
            (uint32_t)V, (uint32_t)(N / 4), (float4*)out);
    return;
  }
  klaunch(k_gather_rows, grid_for(rows * N), 256, 0, st, idx, rows, table, V, N, out);
}

bool scatter_scan_form(int64_t rows, int64_t V) { return scatter_scans(rows, V); }

int64_t scatter_workspace_bytes(int64_t rows, int64_t V, int64_t N) {
  if (scatter_scans(rows, V)) return 0;
  const int64_t items = (rows + kSeg - 1) / kSeg + V;
  const int64_t ints = rows + 2 * (V + 1) + 2 * items;
  return (ints * 4 + 255) / 256 * 256 + items * N * 8;
}

void scatter_rows(const int32_t* idx, int64_t rows, const float* dy, int64_t V, int64_t N, float* out, void* work,
                  hipStream_t st) {
  if (V * N <= 0) return;
  if (V > kMaxBucketV || rows >= (int64_t(1) << 31)) throw std::runtime_error("scatter_rows: V or rows too large");
  if (scatter_scans(rows, V)) {
    const int64_t ny = (N + 255) / 256;
    if (ny > 65535) throw std::runtime_error("scatter_rows: N too large");
    klaunch(k_scatter_scan, dim3((unsigned)V, (unsigned)ny), 256, 0, st, idx, rows, dy, N, out);
    return;
  }
  const int64_t items = (rows + kSeg - 1) / kSeg + V;
  int32_t* perm = static_cast<int32_t*>(work);
  int32_t* offs = perm + rows;
  int32_t* cstart = offs + V + 1;
  int32_t* item_rng = cstart + V + 1;
  const int64_t ints = rows + 2 * (V + 1) + 2 * items;
  double* part = reinterpret_cast<double*>(static_cast<char*>(work) + (ints * 4 + 255) / 256 * 256);
  const int nw = V <= kWaveHistV ? kBucketWaves : 1;
  const int64_t hist_bytes = (int64_t)nw * (V + 1) * 4;
  const int stash = hist_bytes + rows * 4 <= 65536 ? 1 : 0;
  const size_t lds = (size_t)(hist_bytes + (stash ? rows * 4 : 0));
  klaunch(k_bucket_rows, 1, kBucketWaves * 64, lds, st, idx, rows, V, stash, perm, offs, cstart, item_rng);
  const int64_t ny = (N + 255) / 256;
  dim3 g2((unsigned)items, (unsigned)(ny > 64 ? 64 : ny));
  klaunch(k_segment_partials, g2, 256, 0, st, dy, N, V, perm, cstart, item_rng, part);
  klaunch(k_segment_finish, grid_for(V * N), 256, 0, st, part, N, V, cstart, out);
}

}  // namespace tgk
