// Fused causal attention for gfx950: one launch computes, per (batch, head) and block of
// 32 query rows,
//   S  = Q K^T                      (f32 MFMA, 16 x 16 tiles on all eight wavefronts)
//   S2 = f32(S * scale)             (mul_scalar)
//   P  = causal softmax of S2 rows  (f32 exp, f64 row sum, one f64 reciprocal per row)
//   Pd = dropout(P)                 (the reference's hash on the flat [B,H,T,T] index)
//   O  = Pd V                       (f32 MFMA, 16 x 16 tiles, one per wavefront)
// with Q, K, V and S / Pd tiles resident in LDS. P and Pd are written out (the backward
// pass reads them); S and S2 never reach memory. A block of query rows [i0, i0 + 32) reads,
// multiplies and normalises only keys [0, i0 + 32): the causal mask zeroes the rest, and
// P / Pd store exact zeros there. These kernels take dh = 64 with T = 64 or 128; smaller
// heads (T <= 64, dh <= 64: the reference's sample transformers run T = 8 and 16 with
// dh = 16) take a one-workgroup-per-head pair, k_attn_small_fwd / _bwd, at the end of the
// file. Built with -ffp-contract=off.
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
constexpr int kLDV = kDH + 4;  // V rows, read one column per lane: 4 rows apart land 16 banks apart

// v_mfma_f32_16x16x4f32 fragments: A (16 x 4) lane l holds A[l % 16][l / 16], B (4 x 16)
// lane l holds B[l / 16][l % 16], the accumulator lane l register r holds
// D[4 (l / 16) + r][l % 16]. A lane's float4 of k-contiguous operand values feeds four
// consecutive instructions (k = kb + 4 (l / 16) + step), A and B permuted alike.
__device__ __forceinline__ f32x4 mfma16(const f32x4& a, const f32x4& b, f32x4 c) {
#pragma unroll
  for (int s = 0; s < 4; ++s) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], c, 0, 0, 0);
  return c;
}

// Block -> (batch x head, row block). The dispatcher gives a CU the blocks j and j + 32 of
// its XCD (32 CUs each), so the second half of each XCD's blocks walks the row blocks in
// reverse: a CU then holds a long row block (near the end of the sequence, all keys) and
// a short one, instead of two of the same length. The row blocks of one head stay on one
// XCD, whose L2 holds their common K and V.
template <int NRB>
__device__ __forceinline__ void row_block(uint32_t bid, uint32_t nblk, int& bh, int& rb) {
  const uint32_t L = gd::xcd_order(bid, nblk);
  const uint32_t G = nblk % gd::kXcds == 0 ? nblk / gd::kXcds : nblk;   // blocks per XCD (in L order)
  if (G % (2 * NRB) != 0) {
    bh = (int)(L / NRB);
    rb = (int)(L % NRB);
    return;
  }
  const uint32_t x = L / G, j = L % G, half = G / 2;
  if (j < half) {
    bh = (int)(x * (G / NRB) + j / NRB);
    rb = (int)(j % NRB);
  } else {
    bh = (int)(x * (G / NRB) + half / NRB + (j - half) / NRB);
    rb = NRB - 1 - (int)((j - half) % NRB);
  }
}

// Forward, per (batch, head) and block of kQBF query rows. LDS holds two regions: A takes
// the Q tile, then S2 / Pd; B takes K, then V (read into registers with Q and K, written
// once every wave has finished with K). At 54 KiB a CU runs two or three blocks.
template <int T>
__global__ __launch_bounds__(kNT) void k_attn_fwd(const AttnDesc a) {
  constexpr int QB = kQBF;
  constexpr int LDS_ = T + 4;
  constexpr int RA = (QB * kLD > QB * LDS_ ? QB * kLD : QB * LDS_);
  constexpr int RB = (T * kLD > T * kLDV ? T * kLD : T * kLDV);
  __shared__ __attribute__((aligned(16))) float RegA[RA];   // Q, then S2 / Pd
  __shared__ __attribute__((aligned(16))) float RegB[RB];   // K, then V
  float* Qs = RegA;
  float* Ss = RegA;
  float* Ks = RegB;
  float* Vs = RegB;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  constexpr int NRB = T / QB;
  int bh, rb;
  row_block<NRB>(blockIdx.x, gridDim.x, bh, rb);
  const int b = bh / a.H, hd = bh % a.H;
  const int i0 = rb * QB;
  const int nk = i0 + QB;   // keys this block needs

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
      if (row < nk) {
        kv[u] = *reinterpret_cast<const f32x4*>(k + (int64_t)row * a.skj + c4 * 4);
        vv[u] = *reinterpret_cast<const f32x4*>(v + (int64_t)row * a.svj + c4 * 4);
      }
    }
#pragma unroll
    for (int u = 0; u < QC; ++u) {
      const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
      *reinterpret_cast<f32x4*>(Qs + row * kLD + c4 * 4) = qv[u];
    }
#pragma unroll
    for (int u = 0; u < KC; ++u) {
      const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
      if (row < nk) *reinterpret_cast<f32x4*>(Ks + row * kLD + c4 * 4) = kv[u];
    }
  }
  __syncthreads();

  // S = Q K^T on 16 x 16 tiles: tile t = (m-tile t % 2, key tile t / 2), wave w takes t = w,
  // w + 8, ... of the nk / 8 tiles; k in two blocks of 32 added once (blocked accumulation)
  constexpr int MAXT = (QB / 16) * (T / 16) / (kNT / 64);
  f32x4 sacc[MAXT];
  const int ntile = (QB / 16) * (nk / 16);
#pragma unroll
  for (int u = 0; u < MAXT; ++u) {
    const int t = wave + u * (kNT / 64);
#pragma unroll
    for (int r = 0; r < 4; ++r) sacc[u][r] = 0.0f;
    if (t < ntile) {
      const int m0 = (t % (QB / 16)) * 16, n0 = (t / (QB / 16)) * 16;
#pragma unroll
      for (int s = 0; s < kDH / 32; ++s) {
        f32x4 part = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kq = 0; kq < 2; ++kq) {
          const int kb = s * 32 + kq * 16 + g4 * 4;
          const f32x4 av = *reinterpret_cast<const f32x4*>(Qs + (m0 + l16) * kLD + kb);
          const f32x4 bv = *reinterpret_cast<const f32x4*>(Ks + (n0 + l16) * kLD + kb);
          part = mfma16(av, bv, part);
        }
        sacc[u] += part;
      }
    }
  }
  __syncthreads();   // every read of Q and K is done: their regions take S2 and V
#pragma unroll
  for (int u = 0; u < MAXT; ++u) {
    const int t = wave + u * (kNT / 64);
    if (t < ntile) {
      const int m0 = (t % (QB / 16)) * 16, n0 = (t / (QB / 16)) * 16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const unsigned x = fbits(sacc[u][r]);
        Ss[(m0 + g4 * 4 + r) * LDS_ + n0 + l16] =
            a.has_scale ? bitsf(op_eval(FO_MULS, x, 0u, DT_F32, DT_F32, DT_F32, a.scale, 0.0, 0u, 0u, 0u)) : bitsf(x);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < KC; ++u) {
    const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
    if (row < nk) *reinterpret_cast<f32x4*>(Vs + row * kLDV + c4 * 4) = vv[u];
  }
  __syncthreads();

  // Rows: wave w takes rows w * RPW .. + RPW, all in flight; lane l holds columns l + 64 u.
  // Columns past the diagonal hold exact zeros in P and Pd (stored for every column < T).
  {
    constexpr int NU = T / 64;
    constexpr int RPW = QB / (kNT / 64);
    const unsigned seed = a.seed ? (unsigned)*a.seed : 0u;
    // the rows of a wavefront span [i0 + wave * RPW, + RPW): a 64-column chunk past all of
    // their diagonals is skipped by the whole wavefront (its P / Pd columns are zeros)
    const int ilw = __builtin_amdgcn_readfirstlane(wave) * RPW;
    const int nu = min(NU, (i0 + ilw + RPW - 1) / 64 + 1);
    float x[RPW][NU], mx[RPW];
#pragma unroll
    for (int w = 0; w < RPW; ++w) {
      const int il = ilw + w, i = i0 + il;
      mx[w] = bitsf(0xff800000u);
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int col = lane + 64 * u;
        x[w][u] = 0.0f;
        if (u < nu && col <= i) {
          x[w][u] = Ss[il * LDS_ + col];
          mx[w] = fmaxf(mx[w], x[w][u]);
        }
      }
    }
#pragma unroll
    for (int w = 0; w < RPW; ++w) mx[w] = wave_allmax(mx[w]);
    float ex[RPW][NU];
    double sum[RPW];
#pragma unroll
    for (int w = 0; w < RPW; ++w) {
      const int i = i0 + ilw + w;
      sum[w] = 0.0;
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int col = lane + 64 * u;
        ex[w][u] = 0.0f;
        if (u < nu && col <= i) ex[w][u] = expf(x[w][u] - mx[w]);
        sum[w] += (double)ex[w][u];
      }
    }
#pragma unroll
    for (int w = 0; w < RPW; ++w) sum[w] = wave_allsum(sum[w]);
#pragma unroll
    for (int w = 0; w < RPW; ++w) {
      const int il = ilw + w, i = i0 + il;
      const int64_t rflat = (int64_t)bh * T + i;
      const double rs = 1.0 / sum[w];
      unsigned* P = reinterpret_cast<unsigned*>(a.p) + rflat * T;
      unsigned* PD = a.pd ? reinterpret_cast<unsigned*>(a.pd) + rflat * T : nullptr;
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int col = lane + 64 * u;
        unsigned pv = 0u, dv = 0u;
        if (u < nu && col <= i) {
          pv = fbits((float)((double)ex[w][u] * rs));
          dv = a.has_dropout ? dropout_bits(pv, seed, a.salt, a.drop_p, a.drop_scale, (unsigned)(rflat * T + col)) : pv;
        }
        P[col] = pv;
        if (PD) PD[col] = dv;
        if (col < nk) Ss[il * LDS_ + col] = bitsf(dv);
      }
    }
  }
  __syncthreads();

  // O = Pd V: 16 x 16 tiles, one per wavefront (m-tile w / 4, d-tile w % 4), k over the
  // nk keys in blocks of 64 added once
  {
    static_assert((QB / 16) * (kDH / 16) == kNT / 64, "one O tile per wavefront");
    const int m0 = (wave / (kDH / 16)) * 16, n0 = (wave % (kDH / 16)) * 16;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int kb0 = 0; kb0 < nk; kb0 += 64) {
      f32x4 part = {0.0f, 0.0f, 0.0f, 0.0f};
      const int kend = min(nk, kb0 + 64);
      for (int kq = kb0; kq < kend; kq += 16) {
        const int kb = kq + g4 * 4;
        const f32x4 av = *reinterpret_cast<const f32x4*>(Ss + (m0 + l16) * LDS_ + kb);
        f32x4 bv;
#pragma unroll
        for (int s = 0; s < 4; ++s) bv[s] = Vs[(kb + s) * kLDV + n0 + l16];
        part = mfma16(av, bv, part);
      }
      acc += part;
    }
    float* o = a.o + b * a.sob + hd * a.soh;
#pragma unroll
    for (int r = 0; r < 4; ++r) o[(int64_t)(i0 + m0 + g4 * 4 + r) * a.soi + n0 + l16] = acc[r];
  }
}


// Backward, kernel A (per kQBF query rows [i0, i0 + 32), keys [0, i0 + 32)): dPd = dO V^T,
// the dropout and softmax backward row math giving dS (written for those keys, the only
// ones kernel B reads), and dQ = dS K. LDS as in the forward: region A takes dO, then
// dS; region B takes V, then K (read into registers at the start with this block's P and
// Pd rows). The dropout mask comes from the stored Pd: where P > 0, the forward kept an
// element exactly when Pd != 0, and where P = 0 the mask changes no result.
template <int T>
__global__ __launch_bounds__(kNT) void k_attn_bwd_a(const AttnBwdDesc a) {
  constexpr int QB = kQBF;
  constexpr int LDS_ = T + 4;
  constexpr int RA = (QB * kLD > QB * LDS_ ? QB * kLD : QB * LDS_);
  constexpr int RB = (T * kLD > T * kLDV ? T * kLD : T * kLDV);
  __shared__ __attribute__((aligned(16))) float RegA[RA];
  __shared__ __attribute__((aligned(16))) float RegB[RB];
  float* Os = RegA;   // dO rows
  float* Ss = RegA;   // dS
  float* Vs = RegB;
  float* Ks = RegB;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  constexpr int NRB = T / QB;
  int bh, rb;
  row_block<NRB>(blockIdx.x, gridDim.x, bh, rb);
  const int b = bh / a.H, hd = bh % a.H;
  const int i0 = rb * QB, nk = i0 + QB;
  constexpr int NU = T / 64;
  constexpr int RPW = QB / (kNT / 64);   // rows per wavefront in the row math
  const int ilw = __builtin_amdgcn_readfirstlane(wave) * RPW;
  const int nu = min(NU, (nk + 63) / 64);   // 64-column chunks holding keys < nk

  // P and Pd of this wavefront's rows, dO, V and K: every load in flight before the LDS writes
  unsigned pv[RPW][NU], dv0[RPW][NU];
#pragma unroll
  for (int w = 0; w < RPW; ++w) {
    const int64_t rflat = (int64_t)bh * T + i0 + ilw + w;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      pv[w][u] = dv0[w][u] = 0u;
      if (u < nu) {
        pv[w][u] = reinterpret_cast<const unsigned*>(a.p)[rflat * T + lane + 64 * u];
        dv0[w][u] = reinterpret_cast<const unsigned*>(a.pd)[rflat * T + lane + 64 * u];
      }
    }
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
      if (row < nk) {
        vv[u] = *reinterpret_cast<const f32x4*>(v + (int64_t)row * a.svj + c4 * 4);
        kk[u] = *reinterpret_cast<const f32x4*>(k + (int64_t)row * a.skj + c4 * 4);
      }
    }
#pragma unroll
    for (int u = 0; u < QC; ++u) {
      const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
      *reinterpret_cast<f32x4*>(Os + row * kLD + c4 * 4) = ov[u];
    }
#pragma unroll
    for (int u = 0; u < KC; ++u) {
      const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
      if (row < nk) *reinterpret_cast<f32x4*>(Vs + row * kLD + c4 * 4) = vv[u];
    }
  }
  __syncthreads();

  // dPd = dO V^T on 16 x 16 tiles (the forward's S tiling)
  constexpr int MAXT = (QB / 16) * (T / 16) / (kNT / 64);
  f32x4 pacc[MAXT];
  const int ntile = (QB / 16) * (nk / 16);
#pragma unroll
  for (int u = 0; u < MAXT; ++u) {
    const int t = wave + u * (kNT / 64);
#pragma unroll
    for (int r = 0; r < 4; ++r) pacc[u][r] = 0.0f;
    if (t < ntile) {
      const int m0 = (t % (QB / 16)) * 16, n0 = (t / (QB / 16)) * 16;
#pragma unroll
      for (int s = 0; s < kDH / 32; ++s) {
        f32x4 part = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kq = 0; kq < 2; ++kq) {
          const int kb = s * 32 + kq * 16 + g4 * 4;
          const f32x4 av = *reinterpret_cast<const f32x4*>(Os + (m0 + l16) * kLD + kb);
          const f32x4 bv = *reinterpret_cast<const f32x4*>(Vs + (n0 + l16) * kLD + kb);
          part = mfma16(av, bv, part);
        }
        pacc[u] += part;
      }
    }
  }
  __syncthreads();   // every read of dO and V is done: their regions take dPd and K
#pragma unroll
  for (int u = 0; u < MAXT; ++u) {
    const int t = wave + u * (kNT / 64);
    if (t < ntile) {
      const int m0 = (t % (QB / 16)) * 16, n0 = (t / (QB / 16)) * 16;
#pragma unroll
      for (int r = 0; r < 4; ++r) Ss[(m0 + g4 * 4 + r) * LDS_ + n0 + l16] = pacc[u][r];
    }
  }
#pragma unroll
  for (int u = 0; u < KC; ++u) {
    const int c = u * kNT + tid, row = c / (kDH / 4), c4 = c % (kDH / 4);
    if (row < nk) *reinterpret_cast<f32x4*>(Ks + row * kLDV + c4 * 4) = kk[u];
  }
  __syncthreads();

  // dS rows: v0 = dropout(dPd), s = f32(rowsum f32(v0 * P)) (f64 sum), dS = f32((v0 - s) * P)
  // [* scale]: the row-fused group's arithmetic, over the keys < nk (P is zero past the
  // diagonal: those dS are +-0 and nothing reads them beyond nk)
  {
    unsigned v0[RPW][NU];
    double sum[RPW];
#pragma unroll
    for (int w = 0; w < RPW; ++w) {
      const int il = ilw + w;
      sum[w] = 0.0;
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int col = lane + 64 * u;
        v0[w][u] = 0u;
        if (u < nu && col < nk) {
          const unsigned x = fbits(Ss[il * LDS_ + col]);
          v0[w][u] = a.has_dropout ? fbits((float)((double)bitsf(x) * (dv0[w][u] != 0u ? a.drop_scale : 0.0))) : x;
          sum[w] += (double)(bitsf(v0[w][u]) * bitsf(pv[w][u]));
        }
      }
    }
#pragma unroll
    for (int w = 0; w < RPW; ++w) sum[w] = wave_allsum(sum[w]);
#pragma unroll
    for (int w = 0; w < RPW; ++w) {
      const int il = ilw + w;
      const int64_t rflat = (int64_t)bh * T + i0 + il;
      const float sf = (float)(sum[w] / 1.0);
      unsigned* D = reinterpret_cast<unsigned*>(a.ds) + rflat * T;
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int col = lane + 64 * u;
        if (u < nu && col < nk) {
          const unsigned t = fbits((bitsf(v0[w][u]) - sf) * bitsf(pv[w][u]));
          const unsigned d = a.has_scale ? op_eval(FO_MULS, t, 0u, DT_F32, DT_F32, DT_F32, a.scale, 0.0, 0u, 0u, 0u) : t;
          Ss[il * LDS_ + col] = bitsf(d);
          D[col] = d;
        }
      }
    }
  }
  __syncthreads();

  // dQ = dS K: 16 x 16 tiles, one per wavefront, k over the nk keys in blocks of 64
  {
    const int m0 = (wave / (kDH / 16)) * 16, n0 = (wave % (kDH / 16)) * 16;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int kb0 = 0; kb0 < nk; kb0 += 64) {
      f32x4 part = {0.0f, 0.0f, 0.0f, 0.0f};
      const int kend = min(nk, kb0 + 64);
      for (int kq = kb0; kq < kend; kq += 16) {
        const int kb = kq + g4 * 4;
        const f32x4 av = *reinterpret_cast<const f32x4*>(Ss + (m0 + l16) * LDS_ + kb);
        f32x4 bv;
#pragma unroll
        for (int s = 0; s < 4; ++s) bv[s] = Ks[(kb + s) * kLDV + n0 + l16];
        part = mfma16(av, bv, part);
      }
      acc += part;
    }
    float* o = a.dq + b * a.sdqb + hd * a.sdqh;
#pragma unroll
    for (int r = 0; r < 4; ++r) o[(int64_t)(i0 + m0 + g4 * 4 + r) * a.sdqi + n0 + l16] = acc[r];
  }
}

// Transposed slices in LDS: element (m, i) (slice column m, slice row i) sits at
// m ld + (i ^ tswz(m)), ld = R + 16. The XOR moves whole 4-element groups, so a 128-bit
// read of i .. i + 3 (i % 4 == 0) stays one aligned access; with it the transposed 4-byte
// stores (lanes over 8 or 16 columns m and 8 or 4 rows i) and the fragment reads (16
// columns m, 16 rows i) meet no bank twice, where the plain layout (ld = R + 4) put two
// or four store lanes on a bank.
template <int R>
__device__ __forceinline__ int tswz(int m) { return 4 * ((m >> 2) & (R / 4 - 1)); }

// Rows [i0, R) of a COLS-wide slice (row stride rs, 16-byte aligned rows) into registers,
// every load in flight at once; store_t writes them transposed to LDS (column c of the
// slice becomes row c, row i column (i - i0) ^ tswz(c) of a row length `ld`).
template <int R, int COLS>
struct SliceT {
  static constexpr int C = R * COLS / 4 / kNT;
  static_assert(C >= 1 && R * COLS / 4 % kNT == 0, "slice is whole load rounds");
  f32x4 v[C];
  __device__ __forceinline__ void load(const float* src, int64_t rs, int i0, int tid) {
#pragma unroll
    for (int u = 0; u < C; ++u) {
      const int c = u * kNT + tid, row = c / (COLS / 4), c4 = c % (COLS / 4);
      if (row >= i0) v[u] = *reinterpret_cast<const f32x4*>(src + (int64_t)row * rs + c4 * 4);
    }
  }
  __device__ __forceinline__ void store_t(float* dst, int ld, int i0, int tid) const {
#pragma unroll
    for (int u = 0; u < C; ++u) {
      const int c = u * kNT + tid, row = c / (COLS / 4), c4 = c % (COLS / 4);
      if (row >= i0)
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[(c4 * 4 + e) * ld + ((row - i0) ^ tswz<R>(c4 * 4 + e))] = v[u][e];
    }
  }
};

// Backward, kernel B (per KB keys [j0, j0 + 32)): dV = Pd^T dO and dK = dS^T Q over the
// query rows i >= j0 (the causal mask zeroes Pd and dS above the diagonal), 16 x 16 tiles,
// one per wavefront, k over the rows in blocks of 64. LDS holds the slices transposed (key
// rows of Pd / dS, head-dimension rows of dO / Q, rows i in 4-element groups placed by
// tswz): region 1 the Pd
// slice, then the dS slice; region 2 dO, then Q (dS and Q wait in registers while dV is
// formed). The row blocks pair long with short on a CU, as in the forward.
template <int T>
__global__ __launch_bounds__(kNT) void k_attn_bwd_b(const AttnBwdDesc a) {
  constexpr int KB = kQB;
  constexpr int LDT = T + 16;
  __shared__ __attribute__((aligned(16))) float Reg1[KB * LDT];    // Pd^T, then dS^T
  __shared__ __attribute__((aligned(16))) float Reg2[kDH * LDT];   // dO^T, then Q^T

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  constexpr int NJB = T / KB;
  int bh, rbk;
  row_block<NJB>(blockIdx.x, gridDim.x, bh, rbk);
  const int jb = NJB - 1 - rbk;   // row block rb -> key block from the end: long ones pair with short
  const int b = bh / a.H, hd = bh % a.H;
  const int j0 = jb * KB;
  const int mt = T - j0;          // query rows i in [j0, T)
  const int64_t prow = (int64_t)bh * T * T;
  {
    SliceT<T, KB> pd;
    SliceT<T, kDH> od;
    pd.load(a.pd + prow + j0, T, j0, tid);
    od.load(a.dout + b * a.sob + hd * a.soh, a.soi, j0, tid);
    pd.store_t(Reg1, LDT, j0, tid);
    od.store_t(Reg2, LDT, j0, tid);
  }
  SliceT<T, KB> ds;
  SliceT<T, kDH> qq;
  ds.load(a.ds + prow + j0, T, j0, tid);
  qq.load(a.q + b * a.sqb + hd * a.sqh, a.sqi, j0, tid);
  __syncthreads();

  static_assert((KB / 16) * (kDH / 16) == kNT / 64, "one output tile per wavefront");
  const int m0 = (wave / (kDH / 16)) * 16, n0 = (wave % (kDH / 16)) * 16;   // rows: keys j0 + m0, cols: d
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    if (which == 1) {
      __syncthreads();   // dV's reads of both regions are done
      ds.store_t(Reg1, LDT, j0, tid);
      qq.store_t(Reg2, LDT, j0, tid);
      __syncthreads();
    }
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int kb0 = 0; kb0 < mt; kb0 += 64) {
      f32x4 part = {0.0f, 0.0f, 0.0f, 0.0f};
      const int kend = min(mt, kb0 + 64);
      for (int kq = kb0; kq < kend; kq += 16) {
        const int kb = kq + g4 * 4;
        const f32x4 av = *reinterpret_cast<const f32x4*>(Reg1 + (m0 + l16) * LDT + (kb ^ tswz<T>(m0 + l16)));
        const f32x4 bv = *reinterpret_cast<const f32x4*>(Reg2 + (n0 + l16) * LDT + (kb ^ tswz<T>(n0 + l16)));
        part = mfma16(av, bv, part);
      }
      acc += part;
    }
    if (which == 0) {
      float* o = a.dv + b * a.sdvb + hd * a.sdvh;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[(int64_t)(j0 + m0 + g4 * 4 + r) * a.sdvj + n0 + l16] = acc[r];
    } else {
      float* o = a.dk + b * a.sdkb + hd * a.sdkh;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[(int64_t)(j0 + m0 + g4 * 4 + r) * a.sdkj + (int64_t)(n0 + l16) * a.sdkd] = acc[r];
    }
  }
}

// ---- small heads: T <= 64 and dh <= 64 ------------------------------------------------
// One workgroup per (batch, head) holds Q, K, V (and dO) and the T x T rows in LDS. Every
// product accumulates in f64 in increasing k, the evaluator's order (an f32 x f32
// product is exact in f64), and rounds once to f32; entries past the diagonal, which
// the causal mask makes zero, are skipped. The softmax, dropout and softmax-backward row
// arithmetic is the kernels' above, one wavefront per row (a row fits one wavefront).
constexpr int kNTS = 256;
constexpr int kDHM = 64;        // largest head size
constexpr int kLDH = kDHM + 1;  // Q / K / V / dO rows in LDS

bool big_heads(int64_t T, int64_t dh) { return dh == kDH && (T == 64 || T == 128); }

template <int TM>
__global__ __launch_bounds__(kNTS) void k_attn_small_fwd(const AttnDesc a) {
  constexpr int LS = TM + 1;
  __shared__ float Qs[TM * kLDH], Ks[TM * kLDH], Vs[TM * kLDH];
  __shared__ float Ss[TM * LS];   // S2, then Pd
  const int T = a.T, dh = a.dh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int bh = blockIdx.x, b = bh / a.H, hd = bh % a.H;
  {
    const float* q = a.q + b * a.sqb + hd * a.sqh;
    const float* k = a.k + b * a.skb + hd * a.skh;
    const float* v = a.v + b * a.svb + hd * a.svh;
    for (int e = tid; e < T * dh; e += kNTS) {
      const int i = e / dh, d = e % dh;
      Qs[i * kLDH + d] = q[(int64_t)i * a.sqi + d];
      Ks[i * kLDH + d] = k[(int64_t)i * a.skj + d];
      Vs[i * kLDH + d] = v[(int64_t)i * a.svj + d];
    }
  }
  __syncthreads();
  for (int e = tid; e < T * T; e += kNTS) {
    const int i = e / T, j = e % T;
    if (j > i) continue;
    double s = 0.0;
    for (int d = 0; d < dh; ++d) s += (double)Qs[i * kLDH + d] * (double)Ks[j * kLDH + d];
    const unsigned x = fbits((float)s);
    Ss[i * LS + j] = a.has_scale ? bitsf(op_eval(FO_MULS, x, 0u, DT_F32, DT_F32, DT_F32, a.scale, 0.0, 0u, 0u, 0u)) : bitsf(x);
  }
  __syncthreads();
  const unsigned seed = a.seed ? (unsigned)*a.seed : 0u;
  for (int i = wave; i < T; i += kNTS / 64) {
    const int j = lane;
    const bool on = j <= i;
    const float x = on ? Ss[i * LS + j] : 0.0f;
    const float mx = wave_allmax(on ? x : bitsf(0xff800000u));
    const float ex = on ? expf(x - mx) : 0.0f;
    const double rs = 1.0 / wave_allsum((double)ex);
    const int64_t rflat = (int64_t)bh * T + i;
    unsigned pv = 0u, dv = 0u;
    if (on) {
      pv = fbits((float)((double)ex * rs));
      dv = a.has_dropout ? dropout_bits(pv, seed, a.salt, a.drop_p, a.drop_scale, (unsigned)(rflat * T + j)) : pv;
    }
    if (j < T) {
      reinterpret_cast<unsigned*>(a.p)[rflat * T + j] = pv;
      if (a.pd) reinterpret_cast<unsigned*>(a.pd)[rflat * T + j] = dv;
      Ss[i * LS + j] = bitsf(dv);
    }
  }
  __syncthreads();
  float* o = a.o + b * a.sob + hd * a.soh;
  for (int e = tid; e < T * dh; e += kNTS) {
    const int i = e / dh, d = e % dh;
    double s = 0.0;
    for (int j = 0; j <= i; ++j) s += (double)Ss[i * LS + j] * (double)Vs[j * kLDH + d];
    o[(int64_t)i * a.soi + d] = (float)s;
  }
}

template <int TM>
__global__ __launch_bounds__(kNTS) void k_attn_small_bwd(const AttnBwdDesc a) {
  constexpr int LS = TM + 1;
  __shared__ float Qs[TM * kLDH], Ks[TM * kLDH], Vs[TM * kLDH], Os[TM * kLDH];   // Os: dO
  __shared__ float Ps[TM * LS], Ds[TM * LS], Ss[TM * LS];                         // P, Pd, dPd then dS
  const int T = a.T, dh = a.dh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int bh = blockIdx.x, b = bh / a.H, hd = bh % a.H;
  const int64_t prow = (int64_t)bh * T * T;
  {
    const float* q = a.q + b * a.sqb + hd * a.sqh;
    const float* k = a.k + b * a.skb + hd * a.skh;
    const float* v = a.v + b * a.svb + hd * a.svh;
    const float* g = a.dout + b * a.sob + hd * a.soh;
    for (int e = tid; e < T * dh; e += kNTS) {
      const int i = e / dh, d = e % dh;
      Qs[i * kLDH + d] = q[(int64_t)i * a.sqi + d];
      Ks[i * kLDH + d] = k[(int64_t)i * a.skj + d];
      Vs[i * kLDH + d] = v[(int64_t)i * a.svj + d];
      Os[i * kLDH + d] = g[(int64_t)i * a.soi + d];
    }
    for (int e = tid; e < T * T; e += kNTS) {
      const int i = e / T, j = e % T;
      Ps[i * LS + j] = a.p[prow + e];
      Ds[i * LS + j] = a.pd[prow + e];
    }
  }
  __syncthreads();
  for (int e = tid; e < T * T; e += kNTS) {
    const int i = e / T, j = e % T;
    if (j > i) continue;
    double s = 0.0;
    for (int d = 0; d < dh; ++d) s += (double)Os[i * kLDH + d] * (double)Vs[j * kLDH + d];
    Ss[i * LS + j] = (float)s;
  }
  __syncthreads();
  // dS rows: v0 = dropout(dPd), s = f32(rowsum f32(v0 * P)) (f64 sum),
  // dS = f32((v0 - s) * P) [* scale]; zero past the diagonal
  for (int i = wave; i < T; i += kNTS / 64) {
    const int j = lane;
    const bool on = j <= i;
    unsigned v0 = 0u;
    double sum = 0.0;
    if (on) {
      const unsigned x = fbits(Ss[i * LS + j]);
      v0 = a.has_dropout ? fbits((float)((double)bitsf(x) * (fbits(Ds[i * LS + j]) != 0u ? a.drop_scale : 0.0))) : x;
      sum = (double)(bitsf(v0) * Ps[i * LS + j]);
    }
    const float sf = (float)(wave_allsum(sum) / 1.0);
    unsigned dsv = 0u;
    if (on) {
      const unsigned t = fbits((bitsf(v0) - sf) * Ps[i * LS + j]);
      dsv = a.has_scale ? op_eval(FO_MULS, t, 0u, DT_F32, DT_F32, DT_F32, a.scale, 0.0, 0u, 0u, 0u) : t;
    }
    if (j < T) {
      Ss[i * LS + j] = bitsf(dsv);
      reinterpret_cast<unsigned*>(a.ds)[prow + (int64_t)i * T + j] = dsv;
    }
  }
  __syncthreads();
  float* dq = a.dq + b * a.sdqb + hd * a.sdqh;
  float* dk = a.dk + b * a.sdkb + hd * a.sdkh;
  float* dv = a.dv + b * a.sdvb + hd * a.sdvh;
  for (int e = tid; e < T * dh; e += kNTS) {
    const int r = e / dh, d = e % dh;
    double sq = 0.0, sk = 0.0, sv = 0.0;
    for (int j = 0; j <= r; ++j) sq += (double)Ss[r * LS + j] * (double)Ks[j * kLDH + d];       // dQ = dS K
    for (int i = r; i < T; ++i) {
      sk += (double)Ss[i * LS + r] * (double)Qs[i * kLDH + d];                                   // dK = dS^T Q
      sv += (double)Ds[i * LS + r] * (double)Os[i * kLDH + d];                                   // dV = Pd^T dO
    }
    dq[(int64_t)r * a.sdqi + d] = (float)sq;
    dk[(int64_t)r * a.sdkj + (int64_t)d * a.sdkd] = (float)sk;
    dv[(int64_t)r * a.sdvj + d] = (float)sv;
  }
}

}  // namespace

bool attention_supported(int64_t T, int64_t dh) { return big_heads(T, dh) || (T >= 1 && T <= 64 && dh >= 1 && dh <= kDHM); }

void attention_fwd(const AttnDesc& a, hipStream_t st) {
  if (!big_heads(a.T, a.dh)) {
    const int blocks = a.B * a.H;
    if (blocks <= 0) return;
    if (a.T <= 32) klaunch(k_attn_small_fwd<32>, blocks, kNTS, 0, st, a);
    else klaunch(k_attn_small_fwd<64>, blocks, kNTS, 0, st, a);
    return;
  }
  const int blocks = a.B * a.H * (a.T / kQBF);
  if (blocks <= 0) return;
  if (a.T == 128) klaunch(k_attn_fwd<128>, blocks, kNT, 0, st, a);
  else klaunch(k_attn_fwd<64>, blocks, kNT, 0, st, a);
}

void attention_bwd(const AttnBwdDesc& a, hipStream_t st) {
  if (!big_heads(a.T, a.dh)) {
    const int blocks = a.B * a.H;
    if (blocks <= 0) return;
    if (a.T <= 32) klaunch(k_attn_small_bwd<32>, blocks, kNTS, 0, st, a);
    else klaunch(k_attn_small_bwd<64>, blocks, kNTS, 0, st, a);
    return;
  }
  const int blocks = a.B * a.H * (a.T / kQB);
  if (blocks <= 0) return;
  const int blocks_a = a.B * a.H * (a.T / kQBF);
  if (a.T == 128) {
    klaunch(k_attn_bwd_a<128>, blocks_a, kNT, 0, st, a);
    klaunch(k_attn_bwd_b<128>, blocks, kNT, 0, st, a);
  } else {
    klaunch(k_attn_bwd_a<64>, blocks_a, kNT, 0, st, a);
    klaunch(k_attn_bwd_b<64>, blocks, kNT, 0, st, a);
  }
}

}  // namespace tgk
