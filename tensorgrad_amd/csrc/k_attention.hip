// Fused causal attention forward for gfx950: one launch computes, per (batch, head) and
// block of query rows,
//   S  = Q K^T                      (f32 MFMA, blocked accumulation as in k_gemm)
//   S2 = f32(S * scale)             (mul_scalar)
//   P  = causal softmax of S2 rows  (f64 exp / sum, as the row-fused kernels)
//   Pd = dropout(P)                 (the reference's hash on the flat [B,H,T,T] index)
//   O  = Pd V                       (f32 MFMA, blocked accumulation as in k_gemm)
// with Q, K, V and S / Pd tiles resident in LDS. P and Pd are written out (the backward
// pass reads them); S and S2 never reach memory. The MFMA k-order, the accumulation
// blocking (S: stages of 32 k, O: stages of 64 k), the row softmax's lane layout and
// reduction order follow the unfused kernels, so the fused and unfused paths produce the
// same bits. Built with -ffp-contract=off.
#include "kernels.h"

namespace tgk {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kQB = 32;     // keys per block (backward kernel B)
constexpr int kQBF = 32;    // query rows per block (forward, backward kernel A)
constexpr int kNT = 512;    // eight wavefronts: two per SIMD hide each other's latencies
constexpr int kDH = 64;     // head size
constexpr int kLD = kDH + 4;   // k-contiguous tiles (Q, K, S / Pd rows): conflict-free 128-bit reads
constexpr int kLDV = kDH + 8;  // V rows, read one column per lane

// Forward, per (batch, head) and block of kQBF query rows. LDS holds two regions: A takes
// the Q tile, then S2 / Pd, then the O stage-1 partials; B takes K, then V (read into
// registers with Q and K, written once every wave has finished with K). At 54 KiB a CU
// runs three blocks, so one block's loads and stores overlap another's arithmetic. The
// blocks of one (batch, head) share an XCD (and its L2) for their common K and V.
template <int T, int QB>
__global__ __launch_bounds__(kNT) void k_attn_fwd(const AttnDesc a) {
  constexpr int LDS_ = T + 4;
  constexpr int RA = (QB * kLD > QB * LDS_ ? QB * kLD : QB * LDS_);
  constexpr int RB = (T * kLD > T * kLDV ? T * kLD : T * kLDV);
  __shared__ __attribute__((aligned(16))) float RegA[RA];   // Q, then S2 / Pd, then O stage-1 partials
  __shared__ __attribute__((aligned(16))) float RegB[RB];   // K, then V
  float* Qs = RegA;
  float* Ss = RegA;
  float* Ks = RegB;
  float* Vs = RegB;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lrow = lane & 31, h = lane >> 5;
  constexpr int NRB = T / QB;
  const uint32_t L = gd::xcd_order(blockIdx.x, gridDim.x);
  const int bh = L / NRB, rb = L % NRB;
  const int b = bh / a.H, hd = bh % a.H;
  const int i0 = rb * QB;

  constexpr int QC = QB * kDH / 4 / kNT, KC = T * kDH / 4 / kNT;
  static_assert(QC >= 1 && QB * kDH / 4 % kNT == 0, "Q tile is whole load rounds");
  f32x4 vv[KC];
  {
    const float* q = a.q + b * a.sqb + hd * a.sqh;
    const float* k = a.k + b * a.skb + hd * a.skh;
    const float* v = a.v + b * a.svb + hd * a.svh;
    f32x4 qv[QC], kv[KC];
#pragma unroll
    for (int u = 0; u < QC; ++u) {
      const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
      qv[u] = *reinterpret_cast<const f32x4*>(q + (int64_t)(i0 + row) * a.sqi + c4 * 4);
    }
#pragma unroll
    for (int u = 0; u < KC; ++u) {
      const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
      kv[u] = *reinterpret_cast<const f32x4*>(k + (int64_t)row * a.skj + c4 * 4);
      vv[u] = *reinterpret_cast<const f32x4*>(v + (int64_t)row * a.svj + c4 * 4);
    }
#pragma unroll
    for (int u = 0; u < QC; ++u) {
      const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
      *reinterpret_cast<f32x4*>(Qs + row * kLD + c4 * 4) = qv[u];
    }
#pragma unroll
    for (int u = 0; u < KC; ++u) {
      const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
      *reinterpret_cast<f32x4*>(Ks + row * kLD + c4 * 4) = kv[u];
    }
  }
  __syncthreads();

  constexpr int NTILE = (QB / 32) * (T / 32);
  static_assert(NTILE <= kNT / 64, "one S tile per wavefront");
  const int wm = (wave / (T / 32)) * 32, wn = (wave % (T / 32)) * 32;
  f32x16 sacc;
#pragma unroll
  for (int r = 0; r < 16; ++r) sacc[r] = 0.0f;
  if (wave < NTILE) {
#pragma unroll
    for (int s = 0; s < kDH / 32; ++s) {
      f32x16 part;
#pragma unroll
      for (int r = 0; r < 16; ++r) part[r] = 0.0f;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int kb = s * 32 + g * 8 + h * 4;
        const f32x4 av = *reinterpret_cast<const f32x4*>(Qs + (wm + lrow) * kLD + kb);
        const f32x4 bv = *reinterpret_cast<const f32x4*>(Ks + (wn + lrow) * kLD + kb);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) part = __builtin_amdgcn_mfma_f32_32x32x2f32(av[jj], bv[jj], part, 0, 0, 0);
      }
      sacc += part;
    }
  }
  __syncthreads();   // every read of Q and K is done: their regions take S2 and V
  if (wave < NTILE) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = wm + (r / 4) * 8 + h * 4 + (r % 4), col = wn + lrow;
      const unsigned x = fbits(sacc[r]);
      Ss[row * LDS_ + col] =
          a.has_scale ? bitsf(op_eval(FO_MULS, x, 0u, DT_F32, DT_F32, DT_F32, a.scale, 0.0, 0u, 0u, 0u)) : bitsf(x);
    }
  }
#pragma unroll
  for (int u = 0; u < KC; ++u) {
    const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
    *reinterpret_cast<f32x4*>(Vs + row * kLDV + c4 * 4) = vv[u];
  }
  __syncthreads();

  {
    constexpr int V = T >= 128 ? 2 : 1;
    constexpr int RPW = QB / (kNT / 64);   // rows per wavefront
    constexpr int RW = RPW < 4 ? RPW : 4;  // rows in flight per wavefront
    const unsigned seed = a.seed ? (unsigned)*a.seed : 0u;
    for (int rr = 0; rr < RPW; rr += RW) {
      float x[RW][V];
      bool in_row[RW][V];
      float mx[RW];
#pragma unroll
      for (int w = 0; w < RW; ++w) {
        const int il = wave * RPW + rr + w, i = i0 + il;
        mx[w] = bitsf(0xff800000u);
#pragma unroll
        for (int u = 0; u < V; ++u) {
          x[w][u] = Ss[il * LDS_ + lane * V + u];
          in_row[w][u] = lane * V + u <= i;
          if (in_row[w][u]) mx[w] = fmaxf(mx[w], x[w][u]);
        }
      }
#pragma unroll
      for (int w = 0; w < RW; ++w) mx[w] = wave_allmax(mx[w]);
      double ex[RW][V], sum[RW];
#pragma unroll
      for (int w = 0; w < RW; ++w) {
        sum[w] = 0.0;
#pragma unroll
        for (int u = 0; u < V; ++u) {
          ex[w][u] = in_row[w][u] ? exp((double)x[w][u] - (double)mx[w]) : 0.0;
          if (in_row[w][u]) sum[w] += ex[w][u];
        }
      }
#pragma unroll
      for (int w = 0; w < RW; ++w) sum[w] = wave_allsum(sum[w]);
#pragma unroll
      for (int w = 0; w < RW; ++w) {
        const int il = wave * RPW + rr + w, i = i0 + il;
        const int64_t rflat = (int64_t)bh * T + i;
        unsigned pv[V], dv[V];
#pragma unroll
        for (int u = 0; u < V; ++u) {
          pv[u] = in_row[w][u] ? fbits((float)(ex[w][u] / sum[w])) : 0u;
          dv[u] = a.has_dropout ? dropout_bits(pv[u], seed, a.salt, a.drop_p, a.drop_scale,
                                               (unsigned)(rflat * T + lane * V + u))
                                : pv[u];
        }
        unsigned* P = reinterpret_cast<unsigned*>(a.p) + rflat * T + lane * V;
        unsigned* PD = a.pd ? reinterpret_cast<unsigned*>(a.pd) + rflat * T + lane * V : nullptr;
        if (V == 2) {
          typedef unsigned u2 __attribute__((ext_vector_type(2)));
          *reinterpret_cast<u2*>(P) = (u2){pv[0], pv[V - 1]};
          if (PD) *reinterpret_cast<u2*>(PD) = (u2){dv[0], dv[V - 1]};
        } else {
          P[0] = pv[0];
          if (PD) PD[0] = dv[0];
        }
#pragma unroll
        for (int u = 0; u < V; ++u) Ss[il * LDS_ + lane * V + u] = bitsf(dv[u]);
      }
    }
  }
  __syncthreads();

  {
    constexpr int NS = T / 64;
    constexpr int NTO = (QB / 32) * (kDH / 32);
    static_assert(NTO * NS <= kNT / 64, "one O tile stage per wavefront");
    const int tile = wave % NTO, s = wave / NTO;
    const int om = (tile / (kDH / 32)) * 32, on = (tile % (kDH / 32)) * 32;
    f32x16 part;
#pragma unroll
    for (int r = 0; r < 16; ++r) part[r] = 0.0f;
    if (s < NS) {
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const int kb = s * 64 + g * 8 + h * 4;
        const f32x4 av = *reinterpret_cast<const f32x4*>(Ss + (om + lrow) * LDS_ + kb);
        f32x4 bv;
#pragma unroll
        for (int u = 0; u < 4; ++u) bv[u] = Vs[(kb + u) * kLDV + on + lrow];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) part = __builtin_amdgcn_mfma_f32_32x32x2f32(av[jj], bv[jj], part, 0, 0, 0);
      }
    }
    if (NS == 2) {
      __syncthreads();   // every read of Pd is done: region A takes the stage-1 partials
      float* Xs = RegA;
      static_assert(NTO * 16 * 64 <= RA, "exchange fits region A");
      if (s == 1)
#pragma unroll
        for (int r = 0; r < 16; ++r) Xs[(tile * 16 + r) * 64 + lane] = part[r];
      __syncthreads();
      if (s == 0)
#pragma unroll
        for (int r = 0; r < 16; ++r) part[r] = (0.0f + part[r]) + Xs[(tile * 16 + r) * 64 + lane];
    } else if (s == 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) part[r] = 0.0f + part[r];
    }
    if (s == 0) {
      float* o = a.o + b * a.sob + hd * a.soh;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = om + (r / 4) * 8 + h * 4 + (r % 4);
        o[(int64_t)(i0 + row) * a.soi + on + lrow] = part[r];
      }
    }
  }
}


// One 32 x 32 tile, one 64-k stage of a product whose operands are read one column per
// lane from LDS row-major tiles: out(m, n) = sum_k A[k][m] B[k][n] (A rows at a0 + k * lda,
// B rows at b0 + k * ldb), k = 64 s + 8 g + 4 h + jj in the k_gemm order.
__device__ __forceinline__ f32x16 stage_cols(const float* a0, int lda, const float* b0, int ldb, int s, int lrow,
                                             int h) {
  f32x16 part;
#pragma unroll
  for (int r = 0; r < 16; ++r) part[r] = 0.0f;
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const int kb = s * 64 + g * 8 + h * 4;
    f32x4 av, bv;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      av[u] = a0[(kb + u) * lda + lrow];
      bv[u] = b0[(kb + u) * ldb + lrow];
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) part = __builtin_amdgcn_mfma_f32_32x32x2f32(av[jj], bv[jj], part, 0, 0, 0);
  }
  return part;
}

// Backward, kernel A (per kQBF query rows): dPd = dO V^T, the dropout and softmax
// backward row math giving dS (written out), and dQ = dS K. LDS as in the forward:
// region A takes dO, then dPd / dS, then the dQ stage-1 partials; region B takes V, then
// K (read into registers at the start with this block's P rows). 54 KiB: three blocks a CU.
template <int T, int QB>
__global__ __launch_bounds__(kNT) void k_attn_bwd_a(const AttnBwdDesc a) {
  constexpr int LDS_ = T + 4;
  constexpr int RA = (QB * kLD > QB * LDS_ ? QB * kLD : QB * LDS_);
  constexpr int RB = (T * kLD > T * kLDV ? T * kLD : T * kLDV);
  __shared__ __attribute__((aligned(16))) float RegA[RA];
  __shared__ __attribute__((aligned(16))) float RegB[RB];
  float* Os = RegA;   // dO rows
  float* Ss = RegA;   // dPd, then dS
  float* Vs = RegB;
  float* Ks = RegB;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lrow = lane & 31, h = lane >> 5;
  constexpr int NRB = T / QB;
  const uint32_t L = gd::xcd_order(blockIdx.x, gridDim.x);
  const int bh = L / NRB, rb = L % NRB;
  const int b = bh / a.H, hd = bh % a.H;
  const int i0 = rb * QB;
  constexpr int V = T >= 128 ? 2 : 1;
  constexpr int RPW = QB / (kNT / 64);   // rows per wavefront in the row math
  static_assert(RPW >= 1 && RPW <= 4, "the row math keeps every row of a wavefront in flight");

  // P of this wavefront's rows, dO, V and K: every load in flight before the LDS writes
  unsigned pv[RPW][V];
#pragma unroll
  for (int w = 0; w < RPW; ++w) {
    const int64_t rflat = (int64_t)bh * T + i0 + wave * RPW + w;
#pragma unroll
    for (int u = 0; u < V; ++u) pv[w][u] = reinterpret_cast<const unsigned*>(a.p)[rflat * T + lane * V + u];
  }
  constexpr int QC = QB * kDH / 4 / kNT, KC = T * kDH / 4 / kNT;
  static_assert(QC >= 1 && QB * kDH / 4 % kNT == 0, "dO tile is whole load rounds");
  f32x4 kk[KC];
  {
    const float* o = a.dout + b * a.sob + hd * a.soh + (int64_t)i0 * a.soi;
    const float* v = a.v + b * a.svb + hd * a.svh;
    const float* k = a.k + b * a.skb + hd * a.skh;
    f32x4 ov[QC], vv[KC];
#pragma unroll
    for (int u = 0; u < QC; ++u) {
      const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
      ov[u] = *reinterpret_cast<const f32x4*>(o + (int64_t)row * a.soi + c4 * 4);
    }
#pragma unroll
    for (int u = 0; u < KC; ++u) {
      const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
      vv[u] = *reinterpret_cast<const f32x4*>(v + (int64_t)row * a.svj + c4 * 4);
      kk[u] = *reinterpret_cast<const f32x4*>(k + (int64_t)row * a.skj + c4 * 4);
    }
#pragma unroll
    for (int u = 0; u < QC; ++u) {
      const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
      *reinterpret_cast<f32x4*>(Os + row * kLD + c4 * 4) = ov[u];
    }
#pragma unroll
    for (int u = 0; u < KC; ++u) {
      const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
      *reinterpret_cast<f32x4*>(Vs + row * kLD + c4 * 4) = vv[u];
    }
  }
  __syncthreads();

  // dPd = dO V^T (the QK^T kernel's tiles and k-blocking), one tile per wavefront
  constexpr int NTILE = (QB / 32) * (T / 32);
  static_assert(NTILE <= kNT / 64, "one dPd tile per wavefront");
  const int wm = (wave / (T / 32)) * 32, wn = (wave % (T / 32)) * 32;
  f32x16 pacc;
#pragma unroll
  for (int r = 0; r < 16; ++r) pacc[r] = 0.0f;
  if (wave < NTILE) {
#pragma unroll
    for (int s = 0; s < kDH / 32; ++s) {
      f32x16 part;
#pragma unroll
      for (int r = 0; r < 16; ++r) part[r] = 0.0f;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int kb = s * 32 + g * 8 + h * 4;
        const f32x4 av = *reinterpret_cast<const f32x4*>(Os + (wm + lrow) * kLD + kb);
        const f32x4 bv = *reinterpret_cast<const f32x4*>(Vs + (wn + lrow) * kLD + kb);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) part = __builtin_amdgcn_mfma_f32_32x32x2f32(av[jj], bv[jj], part, 0, 0, 0);
      }
      pacc += part;
    }
  }
  __syncthreads();   // every read of dO and V is done: their regions take dPd and K
  if (wave < NTILE)
#pragma unroll
    for (int r = 0; r < 16; ++r) Ss[(wm + (r / 4) * 8 + h * 4 + (r % 4)) * LDS_ + wn + lrow] = pacc[r];
#pragma unroll
  for (int u = 0; u < KC; ++u) {
    const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
    *reinterpret_cast<f32x4*>(Ks + row * kLDV + c4 * 4) = kk[u];
  }
  __syncthreads();

  // dS rows: v0 = dropout(dPd), v1 = v0 * P, s = f32(rowsum v1) (f64, lanes then
  // butterfly), dS = f32((v0 - s) * P * scale): the row-fused group's arithmetic and lanes.
  {
    const unsigned seed = a.seed ? (unsigned)*a.seed : 0u;
    unsigned v0[RPW][V];
    double sum[RPW];
#pragma unroll
    for (int w = 0; w < RPW; ++w) {
      const int il = wave * RPW + w;
      const int64_t rflat = (int64_t)bh * T + i0 + il;
      sum[w] = 0.0;
#pragma unroll
      for (int u = 0; u < V; ++u) {
        const unsigned x = fbits(Ss[il * LDS_ + lane * V + u]);
        v0[w][u] = a.has_dropout ? dropout_bits(x, seed, a.salt, a.drop_p, a.drop_scale,
                                                (unsigned)(rflat * T + lane * V + u))
                                 : x;
        sum[w] += (double)(bitsf(v0[w][u]) * bitsf(pv[w][u]));
      }
    }
#pragma unroll
    for (int w = 0; w < RPW; ++w) sum[w] = wave_allsum(sum[w]);
#pragma unroll
    for (int w = 0; w < RPW; ++w) {
      const int il = wave * RPW + w;
      const int64_t rflat = (int64_t)bh * T + i0 + il;
      const float sf = (float)(sum[w] / 1.0);
      unsigned dv[V];
#pragma unroll
      for (int u = 0; u < V; ++u) {
        const unsigned t = fbits((bitsf(v0[w][u]) - sf) * bitsf(pv[w][u]));
        dv[u] = a.has_scale ? op_eval(FO_MULS, t, 0u, DT_F32, DT_F32, DT_F32, a.scale, 0.0, 0u, 0u, 0u) : t;
        Ss[il * LDS_ + lane * V + u] = bitsf(dv[u]);
      }
      unsigned* D = reinterpret_cast<unsigned*>(a.ds) + rflat * T + lane * V;
      if (V == 2) {
        typedef unsigned u2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u2*>(D) = (u2){dv[0], dv[V - 1]};
      } else {
        D[0] = dv[0];
      }
    }
  }
  __syncthreads();

  // dQ = dS K (the PV kernel's tiles and k-blocking); the stage-1 partials go through
  // region A once every wave has finished reading dS
  {
    constexpr int NS = T / 64;
    constexpr int NTO = (QB / 32) * (kDH / 32);
    static_assert(NTO * NS <= kNT / 64, "one dQ tile stage per wavefront");
    const int tile = wave % NTO, s = wave / NTO;
    const int om = (tile / (kDH / 32)) * 32, on = (tile % (kDH / 32)) * 32;
    f32x16 part;
#pragma unroll
    for (int r = 0; r < 16; ++r) part[r] = 0.0f;
    if (s < NS) {
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const int kb = s * 64 + g * 8 + h * 4;
        const f32x4 av = *reinterpret_cast<const f32x4*>(Ss + (om + lrow) * LDS_ + kb);
        f32x4 bv;
#pragma unroll
        for (int u = 0; u < 4; ++u) bv[u] = Ks[(kb + u) * kLDV + on + lrow];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) part = __builtin_amdgcn_mfma_f32_32x32x2f32(av[jj], bv[jj], part, 0, 0, 0);
      }
    }
    if (NS == 2) {
      __syncthreads();
      float* Xs = RegA;
      static_assert(NTO * 16 * 64 <= RA, "exchange fits region A");
      if (s == 1)
#pragma unroll
        for (int r = 0; r < 16; ++r) Xs[(tile * 16 + r) * 64 + lane] = part[r];
      __syncthreads();
      if (s == 0)
#pragma unroll
        for (int r = 0; r < 16; ++r) part[r] = (0.0f + part[r]) + Xs[(tile * 16 + r) * 64 + lane];
    } else if (s == 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) part[r] = 0.0f + part[r];
    }
    if (s == 0) {
      float* o = a.dq + b * a.sdqb + hd * a.sdqh;
#pragma unroll
      for (int r = 0; r < 16; ++r) o[(int64_t)(i0 + om + (r / 4) * 8 + h * 4 + (r % 4)) * a.sdqi + on + lrow] = part[r];
    }
  }
}

// Rows [0, R) of a COLS-wide slice (row stride rs, 16-byte aligned rows) into registers,
// every load in flight at once; store_slice writes them to LDS rows of `ld` floats.
template <int R, int COLS>
struct Slice {
  static constexpr int C = R * COLS / 4 / kNT;
  static_assert(C >= 1 && R * COLS / 4 % kNT == 0, "slice is whole load rounds");
  f32x4 v[C];
  __device__ __forceinline__ void load(const float* src, int64_t rs, int tid) {
#pragma unroll
    for (int u = 0; u < C; ++u) {
      const int c = u * kNT + tid, row = c / (COLS / 4), c4 = c % (COLS / 4);
      v[u] = *reinterpret_cast<const f32x4*>(src + (int64_t)row * rs + c4 * 4);
    }
  }
  __device__ __forceinline__ void store(float* dst, int ld, int tid) const {
#pragma unroll
    for (int u = 0; u < C; ++u) {
      const int c = u * kNT + tid, row = c / (COLS / 4), c4 = c % (COLS / 4);
      *reinterpret_cast<f32x4*>(dst + row * ld + c4 * 4) = v[u];
    }
  }
};

// Backward, kernel B (per KB keys): dV = Pd^T dO and dK = dS^T Q over all T query rows,
// each as two 64-row stages added in order (the unfused GEMMs' blocking). LDS: region 1
// holds the Pd slice, then the dS slice, region 2 dO, then Q (dS and Q wait in registers
// while dV is formed); the stage-1 partials pass through region 1. 53 KiB: three blocks a
// CU, the blocks of one head on one XCD.
template <int T, int KB>
__global__ __launch_bounds__(kNT) void k_attn_bwd_b(const AttnBwdDesc a) {
  constexpr int LDK = KB + 4;
  __shared__ __attribute__((aligned(16))) float Reg1[T * LDK];   // Pd[i][j0 ..], then dS[i][j0 ..]
  __shared__ __attribute__((aligned(16))) float Reg2[T * kLD];   // dO[i][:], then Q[i][:]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lrow = lane & 31, h = lane >> 5;
  constexpr int NJB = T / KB;
  const uint32_t L = gd::xcd_order(blockIdx.x, gridDim.x);
  const int bh = L / NJB, jb = L % NJB;
  const int b = bh / a.H, hd = bh % a.H;
  const int j0 = jb * KB;
  const int64_t prow = (int64_t)bh * T * T;
  {
    Slice<T, KB> pd;
    Slice<T, kDH> od;
    pd.load(a.pd + prow + j0, T, tid);
    od.load(a.dout + b * a.sob + hd * a.soh, a.soi, tid);
    pd.store(Reg1, LDK, tid);
    od.store(Reg2, kLD, tid);
  }
  Slice<T, KB> ds;
  Slice<T, kDH> qq;
  ds.load(a.ds + prow + j0, T, tid);
  qq.load(a.q + b * a.sqb + hd * a.sqh, a.sqi, tid);
  __syncthreads();

  constexpr int NS = T / 64;
  constexpr int NTO = (KB / 32) * (kDH / 32);
  static_assert(NTO * NS <= kNT / 64, "one output tile stage per wavefront");
  const int tile = wave % NTO, s = wave / NTO;
  const int wm = (tile / (kDH / 32)) * 32, wn = (tile % (kDH / 32)) * 32;   // rows: keys j0 + wm, cols: d
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    if (which == 1) {
      __syncthreads();   // dV's reads of region 1 (partials included) are done
      ds.store(Reg1, LDK, tid);
      qq.store(Reg2, kLD, tid);
      __syncthreads();
    }
    f32x16 part;
#pragma unroll
    for (int r = 0; r < 16; ++r) part[r] = 0.0f;
    if (s < NS) part = stage_cols(Reg1 + wm, LDK, Reg2 + wn, kLD, s, lrow, h);
    if (NS == 2) {
      __syncthreads();   // every read of region 1 is done: it takes the stage-1 partials
      float* Xs = Reg1;
      static_assert(NTO * 16 * 64 <= T * LDK, "exchange fits region 1");
      if (s == 1)
#pragma unroll
        for (int r = 0; r < 16; ++r) Xs[(tile * 16 + r) * 64 + lane] = part[r];
      __syncthreads();
      if (s == 0)
#pragma unroll
        for (int r = 0; r < 16; ++r) part[r] = (0.0f + part[r]) + Xs[(tile * 16 + r) * 64 + lane];
    } else if (s == 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) part[r] = 0.0f + part[r];
    }
    if (s == 0) {
      if (which == 0) {
        float* o = a.dv + b * a.sdvb + hd * a.sdvh;
#pragma unroll
        for (int r = 0; r < 16; ++r) o[(int64_t)(j0 + wm + (r / 4) * 8 + h * 4 + (r % 4)) * a.sdvj + wn + lrow] = part[r];
      } else {
        float* o = a.dk + b * a.sdkb + hd * a.sdkh;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          o[(int64_t)(j0 + wm + (r / 4) * 8 + h * 4 + (r % 4)) * a.sdkj + (int64_t)(wn + lrow) * a.sdkd] = part[r];
      }
    }
  }
}

}  // namespace

bool attention_supported(int64_t T, int64_t dh) { return dh == kDH && (T == 64 || T == 128); }

void attention_fwd(const AttnDesc& a, hipStream_t st) {
  const int blocks = a.B * a.H * (a.T / kQBF);
  if (blocks <= 0) return;
  if (a.T == 128) klaunch(k_attn_fwd<128, kQBF>, blocks, kNT, 0, st, a);
  else klaunch(k_attn_fwd<64, kQBF>, blocks, kNT, 0, st, a);
}

void attention_bwd(const AttnBwdDesc& a, hipStream_t st) {
  const int blocks = a.B * a.H * (a.T / kQB);
  if (blocks <= 0) return;
  const int blocks_a = a.B * a.H * (a.T / kQBF);
  if (a.T == 128) {
    klaunch(k_attn_bwd_a<128, kQBF>, blocks_a, kNT, 0, st, a);
    klaunch(k_attn_bwd_b<128, kQB>, blocks, kNT, 0, st, a);
  } else {
    klaunch(k_attn_bwd_a<64, kQBF>, blocks_a, kNT, 0, st, a);
    klaunch(k_attn_bwd_b<64, kQB>, blocks, kNT, 0, st, a);
  }
}

}  // namespace tgk
