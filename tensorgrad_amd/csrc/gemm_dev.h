// The direct-to-LDS f32 MFMA GEMM tile for gfx950, shared by k_gemm.hip (plain and
// grouped launches) and by the GEMM kernels generated at run time with a fused
// pointwise epilogue (jit.cpp compiles this file as text with hipRTC, so it includes
// nothing under hipRTC and needs no host code). gemm_tile computes one output tile and
// hands every element to an epilogue functor; StoreC writes it to C.
//
#ifndef TG_GEMM_DEV_H
#define TG_GEMM_DEV_H
#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#include <cstdint>
#else
typedef __hip_internal::int64_t int64_t;
typedef __hip_internal::uint64_t uint64_t;
typedef __hip_internal::uint32_t uint32_t;
#endif

namespace tgk {

// C[z][m][n] = sum_k A[z][m][k] * B[z][k][n], f32 MFMA, f32 accumulate.
// Batch index z decomposes as (z / bdiv, z % bdiv) with two strides per operand, so a
// permuted 4-d view [B, H, T, d] is read in place.
struct GemmDesc {
  int64_t M, N, K, batch, bdiv;
  const float* A; int64_t sAz0, sAz1, sAm, sAk;
  const float* B; int64_t sBz0, sBz1, sBk, sBn;
  float* C; int64_t sCz0, sCz1, sCm, sCn;
};

namespace gd {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kXcds = 8;

constexpr int kMaxSeg = 4;

struct GemmArgs {
  GemmDesc d;
  int64_t k_per_split;
  int splits;
  int tiles_n, tiles_m;   // tile grid (per batch and split)
  float* out;             // split-K workspace (splits > 1)
  int64_t sOs, sOz;       // workspace strides (split, batch)
  // Sum of products (SEG kernels): C = sum_s A_s B_s with K = nseg * seg_stages * BK, every
  // segment with its own operand bases and the strides of d (one batch, one split).
  int nseg = 1;
  int seg_stages = 0;
  const float* segA[kMaxSeg] = {};
  const float* segB[kMaxSeg] = {};
  // A as a concatenation along k (CAT kernels): stages below cat_stages read d.A, the rest
  // read catA (row stride catAm, its k from 0); one batch, one split.
  const float* catA = nullptr;
  int64_t catAm = 0;
  int cat_stages = 0;
  // Column partial sums of an epilogue's summed output (Epi::kColSum): row
  // tm * (waves along M) + the wave's M slot, N columns, f64.
  double* colsum = nullptr;
};

// Same fragments and blocked accumulation as k_gemm (k_gemm.hip), but operand tiles travel from
// global memory straight into LDS (global_load_lds_dwordx4: each lane's 16 bytes land at
// wave-base + lane * 16) through a ring of NS stages, so the loads of stages s+1 .. s+NS-1
// are in flight while stage s is multiplied, without staging registers. LDS rows are not
// padded; 16-byte chunks are XOR-swizzled instead so fragment reads stay conflict-free:
//  * k-contiguous operand, rows [r][BK]: chunk c of row r is stored at c ^ swz(r);
//  * row-contiguous operand, rows [k][ROWS]: chunk c of k-row k is stored at
//    c ^ (((k >> 2) & 1) << 3), which puts the two lane halves (k and k + 4) on opposite
//    halves of the banks.
// Used when K (per split) is a multiple of BK, rows of the row-contiguous operand are a
// multiple of 4 and both operands are 16-byte aligned; rows past M / N are read clamped
// to the last row (their results are never stored). Every tile runs eight wavefronts (two
// per SIMD) so one wavefront's barrier wait, partial-sum adds and LDS latency overlap the
// other's MFMAs: 64 x 32 or 32 x 32 wave tiles for tiles with a 128-wide side, two k
// groups of four for 64 x 64 (below).
// Loads address the tile through a wave-uniform base (SGPRs, advanced per stage) plus a
// fixed 32-bit per-lane offset.
constexpr int kLdsBlock = 256;   // floats one wavefront-wide DMA writes (1 KiB)

// DW: the operand's rows need not be 16-byte aligned (a 65-wide matrix): every lane moves
// one 4-byte element (global_load_lds_dword), four times the instructions, into the same
// swizzled LDS layout, so fragment reads do not change.
template <int ROWS, int BK, bool KFAST, int NT, bool DW = false>
struct DTile {
  static constexpr int CPR = KFAST ? BK / 4 : ROWS / 4;   // 16-byte chunks per LDS row
  static constexpr int NCH = ROWS * BK / 4;               // chunks per tile
  static constexpr int PER = (DW ? ROWS * BK : NCH) / NT; // DMA instructions per thread
  static constexpr int SIZE = ROWS * BK;                  // floats
  static_assert((DW ? ROWS * BK : NCH) % NT == 0, "tile must be a whole number of DMA rounds");
  static_assert(KFAST ? (BK == 32 || BK == 64) : ROWS >= 64, "swizzle needs 8 / 16 chunks per row");

  __device__ __forceinline__ static int swz(int lrow) {
    if (KFAST) return BK == 32 ? ((lrow >> 1) & 7) : (lrow & 15);
    return ((lrow >> 2) & 1) << 3;
  }

  // Per-thread byte offsets of this thread's PER chunks (elements, DW) from the tile origin
  // (row r0, k = k0); fixed for the whole k loop. Rows past `rlim` read the last row; k at
  // or past `kv` (a partial last stage) reads k = kv - 1 (whole k rows of a row-contiguous
  // operand; single elements of a DW k-contiguous one), which the tile then zeroes in LDS.
  __device__ __forceinline__ static void offsets(int64_t sr, int64_t sk, int64_t r0, int64_t rlim, int tid,
                                                 uint32_t* off, int kv = BK) {
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int inst = e * (NT / 64) + wave;
      const int P = inst * 64 + lane;
      if (DW) {
        // LDS float P of the tile: undo the chunk swizzle to find its (row, k)
        if (KFAST) {
          const int row = P / BK, rem = P % BK;
          const int k = min((((rem >> 2) ^ swz(row)) << 2) | (rem & 3), kv - 1);
          const int64_t gr = min(r0 + row, rlim - 1) - r0;
          off[e] = (uint32_t)((gr * sr + k) * 4);
        } else {
          const int k = P / ROWS, rem = P % ROWS;
          const int n = (((rem >> 2) ^ swz(k)) << 2) | (rem & 3);
          const int64_t gr = min(r0 + n, rlim - 1) - r0;
          off[e] = (uint32_t)((min(k, kv - 1) * sk + gr) * 4);
        }
        continue;
      }
      const int row = P / CPR, pc = P % CPR;
      const int c = pc ^ swz(row);
      if (KFAST) {
        const int64_t gr = min(r0 + row, rlim - 1) - r0;
        off[e] = (uint32_t)((gr * sr + c * 4) * 4);
      } else {
        const int64_t gr = min(r0 + c * 4, rlim - 4) - r0;
        off[e] = (uint32_t)((min(row, kv - 1) * sk + gr) * 4);
      }
    }
  }

  // Issue this thread's chunks of one stage: global base `gb` (tile origin of the stage,
  // wave-uniform, in SGPRs) plus the 32-bit per-lane offsets; LDS byte address `lds` of the
  // stage's slot and the wave index `wave`, both wave-uniform, so M0 is scalar arithmetic.
  // Each global_load_lds_dwordx4 moves lane l's 16 bytes to M0 + 16 l (a dword load: 4
  // bytes to M0 + 4 l). It is issued from inline assembly so the compiler does not treat it
  // as an LDS write of unknown extent: for such writes it drains every outstanding load
  // before the next LDS read, which would expose the full load latency at every pipeline
  // stage. The kernel orders LDS reads itself (explicit vmcnt waits and barriers). One wait
  // state separates the M0 write from the load.
  __device__ __forceinline__ static void dma(const float* gb, const uint32_t* off, uint32_t lds, int wave) {
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      if (DW) {
        const uint32_t m0v = lds + (uint32_t)((e * (NT / 64) + wave) * 64 * 4);
        asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off[e]), "s"(gb), "{m0}"(m0v));
      } else {
        const uint32_t m0v = lds + (uint32_t)((e * (NT / 64) + wave) * kLdsBlock * 4);
        asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off[e]), "s"(gb), "{m0}"(m0v));
      }
    }
  }

  // Zero the entries of k >= kv in an LDS slot (threads tid of nt).
  __device__ __forceinline__ static void zero_tail(float* L, int kv, int tid, int nt) {
    if (KFAST) {
      for (int P = tid; P < SIZE; P += nt) {
        const int row = P / BK, rem = P % BK;
        if (((((rem >> 2) ^ swz(row)) << 2) | (rem & 3)) >= kv) L[P] = 0.0f;
      }
    } else {
      for (int P = kv * ROWS + tid; P < SIZE; P += nt) L[P] = 0.0f;
    }
  }

  // The 4 consecutive-k values (kb .. kb+3, kb % 4 == 0) of tile row `row`.
  __device__ __forceinline__ static f32x4 frag(const float* L, int row, int kb) {
    if (KFAST) return *reinterpret_cast<const f32x4*>(L + row * BK + (((kb >> 2) ^ swz(row)) << 2));
    f32x4 v;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = kb + u;
      v[u] = L[k * ROWS + ((((row >> 2) ^ swz(k)) << 2) | (row & 3))];
    }
    return v;
  }
};

// s_waitcnt with vmcnt = N and the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// KG = 2 splits the k stages of a tile between two groups of four wavefronts by parity
// (group g multiplies stages g, g + 2, ...; NS slots, NS / 2 per group), for 64 x 64 tiles
// that have no second 32-column or 32-row wave tile to give a second wavefront per SIMD.
// The groups' sums meet at the end as (stages 0, 2, ..) + (stages 1, 3, ..); with two
// stages that is the single group's (0 + stage 0) + stage 1.
// Block b of the launch -> tile number: consecutive tile numbers go to one XCD (the
// hardware deals blocks to the XCDs round-robin), so tiles sharing operand rows or
// columns share an L2.
__device__ __forceinline__ uint32_t xcd_order(uint32_t b, uint32_t nblk) {
  return nblk % kXcds == 0 ? (b % kXcds) * (nblk / kXcds) + b / kXcds : b;
}

// One output tile (tile number b of the problem g).
// ADW / BDW: operand A / B moves one 4-byte element per lane (rows need no alignment).
// KT: the last stage of a split may be partial (K per split not a multiple of BK): its
// loads clamp k to the last valid k and the tile zeroes the rest of the stage in LDS
// before multiplying it (KT needs DW for a k-contiguous operand).
// SEG: a sum of products over k segments (GemmArgs::nseg): stage st reads segment
// st / seg_stages through that segment's own bases; the per-lane offsets, relative to the
// tile origin within a segment, are the same for every segment (shared strides).
// CAT: A (k-contiguous) is a concatenation along k of d.A (whole 16-byte aligned stages,
// stages below g.cat_stages) and g.catA (the rest, rows of any alignment, moved one element
// per lane into the same LDS layout, the partial last stage included). B runs straight
// through all K.
template <int BM, int BN, int BK, int NS, bool AK, bool BKF, int NT, int KG, class Epi, bool BDW = false,
          bool ADW = false, bool KT = false, bool SEG = false, bool CAT = false>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, uint32_t b, const Epi& epi) {
  // per k group: 4 waves 2 x 2; 8 waves 2 x 4 (BN = 128) or 4 x 2
  constexpr int GT = NT / KG;             // threads per k group
  constexpr int NW = GT / 64;
  constexpr int WGM = NW == 8 && BN == 64 ? 4 : 2, WGN = NW / WGM;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  static_assert(TM >= 1 && TN >= 1, "wave tile below 32 x 32");
  static_assert(KG == 1 || (KG == 2 && NS % 2 == 0), "k groups take alternate slots");
  constexpr int NSG = NS / KG;            // slots per k group
  // A group refills a slot right after the barrier that ends its reads of the slot's
  // previous stage, so it needs a second slot to multiply from meanwhile.
  static_assert(NS % KG == 0 && NSG >= 2, "every k group needs at least two ring slots");
  constexpr int NG = BK / 8;
  using TA = DTile<BM, BK, AK, GT, ADW>;
  using TB = DTile<BN, BK, BKF, GT, BDW>;
  static_assert(!KT || ((!AK || ADW || CAT) && (!BKF || BDW)), "a partial k stage needs DW k-contiguous operands");
  static_assert(!CAT || (AK && !ADW && !SEG && KG == 1), "CAT: a k-contiguous, 16-byte A source first");
  // the second source of a CAT tile (its stages issue more loads than PER: the waits below
  // count PER per stage, the fewer, so they wait at least as long as needed)
  using TA2 = DTile<BM, BK, true, GT, true>;
  constexpr int PER = TA::PER + TB::PER;
  static_assert(PER * (NSG - 1) < 64, "too many loads in flight for vmcnt");
  static_assert(!CAT || (TA2::PER + TB::PER) * (NSG - 1) < 64, "too many loads in flight for vmcnt");
  __shared__ __attribute__((aligned(16))) float As[NS * TA::SIZE];   // NS stages of A
  __shared__ __attribute__((aligned(16))) float Bs[NS * TB::SIZE];   // NS stages of B

  const GemmDesc& d = g.d;
  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int kg = __builtin_amdgcn_readfirstlane(tid / GT);   // k group (wave-uniform)
  const int gtid = tid % GT;
  const int wave = gtid / 64;             // wave within the k group
  const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;

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
  const int nst = kbeg < kend ? (int)((kend - kbeg + (KT ? BK - 1 : 0)) / BK) : 0;
  const int ktail = KT && nst > 0 ? (int)(kend - kbeg - (int64_t)(nst - 1) * BK) : BK;   // k of the last stage
  // Operand bases of stage 0 and the per-stage advance, all wave-uniform.
  const float* a0 = A + m0 * (AK ? d.sAm : 1) + kbeg * (AK ? 1 : d.sAk);
  const float* b0 = B + n0 * (BKF ? d.sBn : 1) + kbeg * (BKF ? 1 : d.sBk);
  const int64_t a_step = AK ? BK : BK * d.sAk, b_step = BKF ? BK : BK * d.sBk;
  uint32_t offa[TA::PER], offb[TB::PER];
  TA::offsets(d.sAm, d.sAk, m0, d.M, gtid, offa);
  TB::offsets(d.sBn, d.sBk, n0, d.N, gtid, offb);
  uint32_t offat[KT && !CAT ? TA::PER : 1], offbt[KT ? TB::PER : 1];   // the partial last stage
  if (KT) {
    if (!CAT) TA::offsets(d.sAm, d.sAk, m0, d.M, gtid, offat, ktail);
    TB::offsets(d.sBn, d.sBk, n0, d.N, gtid, offbt, ktail);
  }
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t lds_a = (uint32_t)(unsigned long)((__attribute__((address_space(3))) float*)As);
  const uint32_t lds_b = (uint32_t)(unsigned long)((__attribute__((address_space(3))) float*)Bs);
  auto issue = [&](int st) {
    const int slot = st % NS;
    if (SEG) {   // one batch, one split: kbeg = 0, z = 0
      const int sg = st / g.seg_stages, sl = st - sg * g.seg_stages;
      const float* sa = sg == 0 ? g.segA[0] : sg == 1 ? g.segA[1] : sg == 2 ? g.segA[2] : g.segA[3];
      const float* sb = sg == 0 ? g.segB[0] : sg == 1 ? g.segB[1] : sg == 2 ? g.segB[2] : g.segB[3];
      TA::dma(sa + m0 * (AK ? d.sAm : 1) + sl * a_step, offa, lds_a + slot * TA::SIZE * 4, wv);
      TB::dma(sb + n0 * (BKF ? d.sBn : 1) + sl * b_step, offb, lds_b + slot * TB::SIZE * 4, wv);
      return;
    }
    if (CAT && st >= g.cat_stages) {   // one split: kbeg = 0
      const float* sa = g.catA + m0 * g.catAm + (int64_t)(st - g.cat_stages) * BK;
      const bool tail = KT && st == nst - 1 && ktail < BK;
      // The second source's per-lane offsets are computed here, for its few stages, from
      // values the compiler cannot see through, so no part of them is hoisted out of the k
      // loop and held in registers across it (that would cost a block per CU).
      int kv = tail ? ktail : BK;
      int t2 = gtid;
      asm volatile("" : "+s"(kv), "+v"(t2));
      uint32_t o2[TA2::PER];
      TA2::offsets(g.catAm, 1, m0, d.M, t2, o2, kv);
      TA2::dma(sa, o2, lds_a + slot * TA::SIZE * 4, wv);
      if (tail) TB::dma(b0 + st * b_step, offbt, lds_b + slot * TB::SIZE * 4, wv);
      else TB::dma(b0 + st * b_step, offb, lds_b + slot * TB::SIZE * 4, wv);
      return;
    }
    if (!CAT && KT && st == nst - 1 && ktail < BK) {
      TA::dma(a0 + st * a_step, offat, lds_a + slot * TA::SIZE * 4, wv);
      TB::dma(b0 + st * b_step, offbt, lds_b + slot * TB::SIZE * 4, wv);
      return;
    }
    TA::dma(a0 + st * a_step, offa, lds_a + slot * TA::SIZE * 4, wv);
    TB::dma(b0 + st * b_step, offb, lds_b + slot * TB::SIZE * 4, wv);
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int lrow = lane % 32, h = lane / 32;
  // this group's stages are kg, kg + KG, ...; it keeps NSG - 1 of them in flight
#pragma unroll
  for (int p = 0; p < NSG - 1; ++p)
    if (kg + p * KG < nst) issue(kg + p * KG);

  const int nit = (nst + KG - 1) / KG;
  const int mine = nst > kg ? (nst - 1 - kg) / KG : -1;   // this group's last iteration
  for (int it = 0; it < nit; ++it) {
    const int st = it * KG + kg;
    // Stage st has landed once at most (own stages issued after it) * PER loads are pending.
    const int after = min(NSG - 2, mine - it);
    if (NSG >= 4 && after >= 3) wait_vmcnt<(NSG >= 4 ? 3 : 0) * PER>();
    else if (NSG >= 3 && after >= 2) wait_vmcnt<(NSG >= 3 ? 2 : 0) * PER>();
    else if (after >= 1) wait_vmcnt<PER>();
    else wait_vmcnt<0>();
    // A bare workgroup barrier: __syncthreads() would also drain every outstanding load
    // (the stages still in flight). The empty asm statements keep the compiler from
    // moving LDS accesses across it; each wave has already waited for its own copies of
    // stage st, and its reads of the slot about to be refilled were consumed by the MFMAs
    // of its group's previous stage.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (KT && ktail < BK && it == (nst - 1) / KG) {
      // The partial last stage has landed (every wave waited for its own copies before the
      // barrier): the whole block zeroes its k >= ktail entries, then meets again. The
      // condition is the same in every thread.
      const int ts = (nst - 1) % NS;
      TA::zero_tail(As + ts * TA::SIZE, ktail, tid, NT);
      TB::zero_tail(Bs + ts * TB::SIZE, ktail, tid, NT);
      __syncthreads();
    }
    if (st >= nst) continue;              // the other group's last stage (odd count)
    if (st + (NSG - 1) * KG < nst) issue(st + (NSG - 1) * KG);
    const float* Ac = As + (st % NS) * TA::SIZE;
    const float* Bc = Bs + (st % NS) * TB::SIZE;
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
      if (grp + 1 < NG) {
        const int kb = (grp + 1) * 8 + h * 4;
#pragma unroll
        for (int i = 0; i < TM; ++i) av[c ^ 1][i] = TA::frag(Ac, wm0 + i * 32 + lrow, kb);
#pragma unroll
        for (int j = 0; j < TN; ++j) bv[c ^ 1][j] = TB::frag(Bc, wn0 + j * 32 + lrow, kb);
      }
      // keep the next group's LDS reads ahead of this group's MFMAs
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            part[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[c][i][jj], bv[c][j][jj], part[i][j], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] += part[i][j];
  }

  if (KG == 2) {
    // group 1 hands its sums to group 0 through LDS (the A ring, free after the barrier)
    static_assert(KG == 1 || NW * TM * TN * 16 * 64 <= NS * TA::SIZE, "exchange fits the A ring");
    __syncthreads();
    float* X = As;
    if (kg == 1) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) X[(((wave * TM + i) * TN + j) * 16 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (kg == 1) return;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] += X[(((wave * TM + i) * TN + j) * 16 + r) * 64 + lane];
  }

  if (g.splits > 1) {   // split-K partial tile into the workspace
    float* O = g.out + split * g.sOs + zz * g.sOz;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t gn = n0 + wn0 + j * 32 + lrow;
        if (gn >= d.N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t gm = m0 + wm0 + i * 32 + (r / 4) * 8 + h * 4 + (r % 4);
          if (gm < d.M) O[gm * d.N + gn] = acc[i][j][r];
        }
      }
    return;
  }
  if constexpr (Epi::kPrefetch) {
    // An epilogue that reads other tensors: every one of its loads for the wave's
    // accumulator values is issued first (clamped to an element in range), then the values
    // are computed and stored. Interleaved, each load would wait for the stores before it
    // (the outputs may alias the inputs as far as the compiler knows): one memory latency
    // per value.
    typename Epi::Pre pre[TM][TN][16];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t gn = min((int64_t)(n0 + wn0 + j * 32 + lrow), d.N - 1);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t gm = min((int64_t)(m0 + wm0 + i * 32 + (r / 4) * 8 + h * 4 + (r % 4)), d.M - 1);
          pre[i][j][r] = epi.load(d, gm, gn);
        }
      }
    if constexpr (Epi::kColSum) {
      // The epilogue also returns the value of an output whose column sums are wanted: each
      // lane totals its column over the wave's rows it holds (f64, in (i, r) order), the two
      // lane halves (h = 0, 1: the other rows of the same column) are added, and lanes of
      // h = 0 store the wave's partial row (one batch: z = 0).
      double cs[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j) cs[j] = 0.0;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int64_t gn = n0 + wn0 + j * 32 + lrow;
          if (gn >= d.N) continue;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int64_t gm = m0 + wm0 + i * 32 + (r / 4) * 8 + h * 4 + (r % 4);
            if (gm < d.M) cs[j] += (double)epi(d, z0, z1, gm, gn, acc[i][j][r], pre[i][j][r]);
          }
        }
      const int64_t prow = (int64_t)tm * WGM + wave / WGN;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const double t = cs[j] + __shfl_xor(cs[j], 32);
        const int64_t gn = n0 + wn0 + j * 32 + lrow;
        if (h == 0 && gn < d.N) g.colsum[prow * d.N + gn] = t;
      }
      return;
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
          if (gm < d.M) epi(d, z0, z1, gm, gn, acc[i][j][r], pre[i][j][r]);
        }
      }
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t gn = n0 + wn0 + j * 32 + lrow;
        if (gn >= d.N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t gm = m0 + wm0 + i * 32 + (r / 4) * 8 + h * 4 + (r % 4);
          if (gm < d.M) epi(d, z0, z1, gm, gn, acc[i][j][r]);
        }
      }
  }
}

// The plain epilogue: element (z, gm, gn) of the product to C.
struct StoreC {
  static constexpr bool kPrefetch = false;
  static constexpr bool kColSum = false;
  __device__ __forceinline__ void operator()(const GemmDesc& d, int64_t z0, int64_t z1, int64_t gm, int64_t gn,
                                             float v) const {
    d.C[z0 * d.sCz0 + z1 * d.sCz1 + gm * d.sCm + gn * d.sCn] = v;
  }
};


// ---- skinny products (the layout and the choice are described in k_gemm.hip) ----------
// GemmArgs as: tiles_m = row blocks of 16, tiles_n = column blocks of NT x 16, splits and
// k_per_split the k ranges, out the split partials [split][M][N].
constexpr int kSkinnySteps = 4;   // 16-k steps per wavefront per batch

__device__ __forceinline__ f32x4 mfma16x4(const f32x4& a, const f32x4& b, f32x4 c) {
#pragma unroll
  for (int s = 0; s < 4; ++s) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], c, 0, 0, 0);
  return c;
}

// Zero outside the operand as a bit mask on a value loaded unconditionally (from a clamped
// address): a select would let the compiler move each load under a branch of its own and
// wait for it there, one memory latency per element.
__device__ __forceinline__ unsigned mask_if(bool keep) { return 0u - (unsigned)keep; }
__device__ __forceinline__ float masked(float v, unsigned keep) { return __uint_as_float(__float_as_uint(v) & keep); }


template <int NT, bool AV, class Epi>
__device__ __forceinline__ void skinny_tile(const GemmArgs& s, const Epi& epi) {
  constexpr int SB = kSkinnySteps;
  __shared__ float red[4 * NT * 256];
  const GemmDesc& d = s.d;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g4 = lane >> 4;
  // consecutive row blocks (which share A's cache lines when A has unit row stride) on
  // one XCD
  const int bid = (int)xcd_order(blockIdx.x, gridDim.x);
  const int rbk = bid % s.tiles_m, rest = bid / s.tiles_m;
  const int cbk = rest % s.tiles_n, sp = rest / s.tiles_n;
  const int M = (int)d.M, N = (int)d.N, K = (int)d.K;
  const int sAm = (int)d.sAm, sAk = (int)d.sAk, sBk = (int)d.sBk, sBn = (int)d.sBn;
  const int kbeg = sp * (int)s.k_per_split, kend = min(K, kbeg + (int)s.k_per_split);
  const int m = rbk * 16 + l16;
  const bool mok = m < M;
  const float* arow = d.A + (mok ? m : M - 1) * sAm;
  bool nok[NT];
  const float* bcol[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n = cbk * NT * 16 + t * 16 + l16;
    nok[t] = n < N;
    bcol[t] = d.B + (nok[t] ? n : N - 1) * sBn;
  }
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  for (int k0 = kbeg; k0 < kend; k0 += 64 * SB) {
    // every load of the batch is issued before any is used (the scheduling barrier keeps
    // the compiler from interleaving waits with the loads)
    f32x4 a[SB];
    f32x4 b[SB][NT];
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const int kb = k0 + (j * 4 + wave) * 16 + g4 * 4;
      if (AV) {
        a[j] = *reinterpret_cast<const f32x4*>(arow + min(kb, kend - 4));
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) a[j][q] = arow[min(kb + q, kend - 1) * sAk];
      }
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) b[j][t][q] = bcol[t][min(kb + q, kend - 1) * sBk];
    }
    __builtin_amdgcn_sched_barrier(0);
    f32x4 part[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) part[t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    // steps past the range multiply zeros (a branch around them would let the compiler
    // sink their loads into it)
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const int kb = k0 + (j * 4 + wave) * 16 + g4 * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) a[j][q] = masked(a[j][q], mask_if(mok && kb + q < kend));
#pragma unroll
      for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int q = 0; q < 4; ++q) b[j][t][q] = masked(b[j][t][q], mask_if(nok[t] && kb + q < kend));
        part[t] = mfma16x4(a[j], b[j][t], part[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] += part[t];
  }
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[(wave * NT + t) * 256 + (g4 * 4 + r) * 16 + l16] = acc[t][r];
  __syncthreads();
  if constexpr (Epi::kPrefetch) {
    // a generated epilogue (one split): the group's loads for the thread's NT outputs
    // first (clamped in range), then the arithmetic and stores
    typename Epi::Pre pre[NT];
#pragma unroll
    for (int q = 0; q < NT; ++q) {
      const int e = tid + q * 256, rc = e % 256;
      pre[q] = epi.load(d, min(rbk * 16 + rc / 16, M - 1), min(cbk * NT * 16 + (e / 256) * 16 + rc % 16, N - 1));
    }
#pragma unroll
    for (int q = 0; q < NT; ++q) {
      const int e = tid + q * 256;
      const float v = ((red[e] + red[NT * 256 + e]) + red[2 * NT * 256 + e]) + red[3 * NT * 256 + e];
      const int t = e / 256, rc = e % 256;
      const int gm = rbk * 16 + rc / 16, gn = cbk * NT * 16 + t * 16 + rc % 16;
      if (gm < M && gn < N) epi(d, 0, 0, gm, gn, v, pre[q]);
    }
    return;
  }
  const int64_t MN = d.M * d.N;
  for (int e = tid; e < NT * 256; e += 256) {
    const float v = ((red[e] + red[NT * 256 + e]) + red[2 * NT * 256 + e]) + red[3 * NT * 256 + e];
    const int t = e / 256, rc = e % 256;
    const int gm = rbk * 16 + rc / 16, gn = cbk * NT * 16 + t * 16 + rc % 16;
    if (gm >= M || gn >= N) continue;
    if (s.splits > 1) s.out[sp * MN + (int64_t)gm * N + gn] = v;
    else d.C[gm * d.sCm + gn * d.sCn] = v;
  }
}


// Small degenerate products (one of M, N, K is 1: outer products and matrix-vector
// products; the small MLP's one-wide layers): a 64 x 64 MFMA tile would compute one real
// row or column, and its fixed cost (operand staging, the k-group exchange) dominates. Each
// output takes L lanes (L divides 64, about K / 8 terms per lane): lane j adds terms
// k = j, j + L, ... in order with f32 FMAs from +0, then an xor butterfly over the L lanes
// combines them, a fixed order. With K = 1 that is f32(0 + a b), the MFMA tile's bits;
// otherwise the rounding of another summation order. A generated epilogue (kPrefetch)
// takes the sum in the lane that would store it (one batch).
template <int L, class Epi>
__device__ __forceinline__ void tiny_tile(const GemmArgs& g, const Epi& epi) {
  const GemmDesc& d = g.d;
  constexpr int kPerBlock = 256 / L;
  const int64_t total = d.M * d.N * d.batch;
  const int lj = (int)threadIdx.x % L;
  // the loop bound is the same in every thread: all lanes reach the butterfly together
  for (int64_t e0 = (int64_t)blockIdx.x * kPerBlock; e0 < total; e0 += (int64_t)gridDim.x * kPerBlock) {
    const int64_t e = e0 + threadIdx.x / L;
    float acc = 0.0f;
    int64_t ci = -1, m = 0, n = 0, z0 = 0, z1 = 0;
    if (e < total) {
      n = e % d.N;
      const int64_t t = e / d.N;
      m = t % d.M;
      const int64_t z = t / d.M;
      z0 = z / d.bdiv;
      z1 = z % d.bdiv;
      const float* a = d.A + z0 * d.sAz0 + z1 * d.sAz1 + m * d.sAm;
      const float* b = d.B + z0 * d.sBz0 + z1 * d.sBz1 + n * d.sBn;
      for (int64_t k = lj; k < d.K; k += L) acc = fmaf(a[k * d.sAk], b[k * d.sBk], acc);
      ci = z0 * d.sCz0 + z1 * d.sCz1 + m * d.sCm + n * d.sCn;
    }
#pragma unroll
    for (int o = L / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (lj == 0 && ci >= 0) {
      if constexpr (Epi::kPrefetch) epi(d, z0, z1, m, n, acc, epi.load(d, m, n));
      else d.C[ci] = acc;
    }
  }
}

// Short products (K at most 16, many outputs: C4's head input gradient [65536, 4] x
// [4, 256]), where a 32-k MFMA stage would be mostly padding and the output is the traffic.
// Block b of tiles_n x tiles_m x batch takes RM rows and 256 columns: thread t keeps column
// 256 bn + t of B in registers, the block's rows of A sit in LDS, and each output is an f32
// FMA chain from +0 in increasing k, four rows' chains side by side, stored as they finish
// (consecutive threads, consecutive columns). Both operands are padded with zeros from K to
// KB: a chain starts at +0 and so never holds -0, and adding +0 to it changes no bit.
// Operand loads are unconditional, from a clamped index, and masked after: a select would
// let the compiler move each load into a branch with its own wait.
// An epilogue that reads other tensors (kPrefetch) has the thread's loads for its RM
// outputs issued first; with kColSum the thread also writes its column's total over the
// block's rows (f64, in row order) to g.colsum[bm * N + n] (one batch).
template <int RM, int KB, class Epi>
__device__ __forceinline__ void smallk_tile(const GemmArgs& g, const Epi& epi) {
  static_assert(RM % 4 == 0 && KB % 4 == 0, "rows in fours, k in fours");
  __shared__ __attribute__((aligned(16))) float As[RM * KB];
  const GemmDesc& d = g.d;
  const int nblk_n = g.tiles_n, nblk_m = g.tiles_m;
  const int64_t blk = blockIdx.x;
  const int bn = (int)(blk % nblk_n);
  const int64_t rest = blk / nblk_n;
  const int bm = (int)(rest % nblk_m);
  const int64_t z = rest / nblk_m;
  const int64_t z0 = z / d.bdiv, z1 = z % d.bdiv;
  const int K = (int)d.K;
  const int64_t m0 = (int64_t)bm * RM, n = (int64_t)bn * 256 + threadIdx.x;
  const float* A = d.A + z0 * d.sAz0 + z1 * d.sAz1;
  const float* B = d.B + z0 * d.sBz0 + z1 * d.sBz1;
  const int rows = (int)min((int64_t)RM, d.M - m0);
  auto keep = [](float v, bool ok) { return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) & (ok ? ~0u : 0u)); };
  for (int e = threadIdx.x; e < RM * KB; e += 256) {
    const int r = e / KB, k = e % KB;
    const float v = A[(m0 + min(r, rows - 1)) * d.sAm + (int64_t)min(k, K - 1) * d.sAk];
    As[e] = keep(v, r < rows && k < K);
  }
  const bool on = n < d.N;
  const float* bc = B + (on ? n : 0) * d.sBn;
  float b[KB];
#pragma unroll
  for (int k = 0; k < KB; ++k) b[k] = keep(bc[(int64_t)min(k, K - 1) * d.sBk], on && k < K);
  __syncthreads();
  if (!on) return;
  auto four_rows = [&](int r, float* acc) {
#pragma unroll
    for (int k = 0; k < KB; k += 4) {
      f32x4 a4[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) a4[j] = *reinterpret_cast<const f32x4*>(As + (r + j) * KB + k);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = fmaf(a4[j][u], b[k + u], acc[j]);
      asm volatile("" ::: "memory");   // one step's LDS reads at a time
    }
  };
  if constexpr (Epi::kPrefetch) {
    typename Epi::Pre pre[RM];
#pragma unroll
    for (int r = 0; r < RM; ++r) pre[r] = epi.load(d, m0 + min(r, rows - 1), n);
    double cs = 0.0;
#pragma unroll
    for (int r = 0; r < RM; r += 4) {
      if (r >= rows) break;
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      four_rows(r, acc);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (r + j < rows) {
          if constexpr (Epi::kColSum) cs += (double)epi(d, z0, z1, m0 + r + j, n, acc[j], pre[r + j]);
          else epi(d, z0, z1, m0 + r + j, n, acc[j], pre[r + j]);
        }
    }
    if constexpr (Epi::kColSum) g.colsum[(int64_t)bm * d.N + n] = cs;
  } else {
    float* C = d.C + z0 * d.sCz0 + z1 * d.sCz1 + n * d.sCn;
    for (int r = 0; r < rows; r += 4) {
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      four_rows(r, acc);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (r + j < rows) C[(m0 + r + j) * d.sCm] = acc[j];
    }
  }
}

}  // namespace gd
}  // namespace tgk

#endif  // TG_GEMM_DEV_H
