// Fused causal attention forward for gfx950: one launch computes, per (batch, head) and
// block of 64 query rows,
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

constexpr int kQB = 64;     // query rows per block
constexpr int kNT = 512;    // eight wavefronts: two per SIMD hide each other's latencies
constexpr int kDH = 64;     // head size
constexpr int kLD = kDH + 4;   // k-contiguous tiles (Q, K, S / Pd rows): conflict-free 128-bit reads
constexpr int kLDV = kDH + 8;  // V rows, read one column per lane

template <int T>
__global__ __launch_bounds__(kNT) void k_attn_fwd(const AttnDesc a) {
  constexpr int LDS_ = T + 4;
  __shared__ __attribute__((aligned(16))) float Qs[kQB * kLD];
  __shared__ __attribute__((aligned(16))) float Ks[T * kLD];
  __shared__ __attribute__((aligned(16))) float Vs[T * kLDV];
  __shared__ __attribute__((aligned(16))) float Ss[kQB * LDS_];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lrow = lane & 31, h = lane >> 5;
  constexpr int RB = T / kQB;
  const int bh = blockIdx.x / RB, rb = blockIdx.x % RB;
  const int b = bh / a.H, hd = bh % a.H;
  const int i0 = rb * kQB;

  // ---- operand tiles: every load in flight before the LDS writes ----
  {
    const float* q = a.q + b * a.sqb + hd * a.sqh;
    const float* k = a.k + b * a.skb + hd * a.skh;
    const float* v = a.v + b * a.svb + hd * a.svh;
    constexpr int QC = kQB * kDH / 4 / kNT, KC = T * kDH / 4 / kNT;
    f32x4 qv[QC], kv[KC], vv[KC];
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
      *reinterpret_cast<f32x4*>(Vs + row * kLDV + c4 * 4) = vv[u];
    }
  }
  __syncthreads();

  // ---- S2 = f32(Q K^T * scale) into Ss: 2 x T/32 tiles of 32 x 32, dealt round-robin to
  // the eight wavefronts ----
  {
    constexpr int NTILE = 2 * (T / 32);
    for (int t = wave; t < NTILE; t += kNT / 64) {
      const int wm = (t / (T / 32)) * 32, wn = (t % (T / 32)) * 32;
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
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
        acc += part;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = wm + (r / 4) * 8 + h * 4 + (r % 4), col = wn + lrow;
        const unsigned x = fbits(acc[r]);
        Ss[row * LDS_ + col] =
            a.has_scale ? bitsf(op_eval(FO_MULS, x, 0u, DT_F32, DT_F32, DT_F32, a.scale, 0.0, 0u, 0u, 0u)) : bitsf(x);
      }
    }
  }
  __syncthreads();

  // ---- causal softmax and dropout, one wavefront per row: lane owns V consecutive
  // columns (the row-fused kernels' layout for D = T). Each wavefront runs four of its
  // rows side by side so their shuffle and exp latencies overlap. ----
  {
    constexpr int V = T >= 128 ? 2 : 1;
    constexpr int RW = 4;   // rows in flight per wavefront
    const unsigned seed = a.seed ? (unsigned)*a.seed : 0u;
    constexpr int RPW = kQB / (kNT / 64);   // rows per wavefront
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
      for (int o = 32; o > 0; o >>= 1)
#pragma unroll
        for (int w = 0; w < RW; ++w) mx[w] = fmaxf(mx[w], __shfl_xor(mx[w], o, 64));
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
      for (int o = 32; o > 0; o >>= 1)
#pragma unroll
        for (int w = 0; w < RW; ++w) sum[w] += __shfl_xor(sum[w], o, 64);
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

  // ---- O = Pd V: four 32 x 32 tiles; with T = 128 the two 64-k stages of a tile go to
  // two wavefronts and are added in stage order, (0 + stage 0) + stage 1 ----
  {
    __shared__ __attribute__((aligned(16))) float Xs[4 * 16 * 64];   // stage-1 partials
    constexpr int NS = T / 64;
    const int tile = wave & 3, s = wave >> 2;
    const int wm = (tile >> 1) * 32, wn = (tile & 1) * 32;
    f32x16 part;
#pragma unroll
    for (int r = 0; r < 16; ++r) part[r] = 0.0f;
    if (s < NS) {
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const int kb = s * 64 + g * 8 + h * 4;
        const f32x4 av = *reinterpret_cast<const f32x4*>(Ss + (wm + lrow) * LDS_ + kb);
        f32x4 bv;
#pragma unroll
        for (int u = 0; u < 4; ++u) bv[u] = Vs[(kb + u) * kLDV + wn + lrow];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) part = __builtin_amdgcn_mfma_f32_32x32x2f32(av[jj], bv[jj], part, 0, 0, 0);
      }
    }
    if (NS == 2 && s == 1)
#pragma unroll
      for (int r = 0; r < 16; ++r) Xs[(tile * 16 + r) * 64 + lane] = part[r];
    __syncthreads();
    if (s == 0) {
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.0f + part[r];
      if (NS == 2)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] += Xs[(tile * 16 + r) * 64 + lane];
      float* o = a.o + b * a.sob + hd * a.soh;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = wm + (r / 4) * 8 + h * 4 + (r % 4);
        o[(int64_t)(i0 + row) * a.soi + wn + lrow] = acc[r];
      }
    }
  }
}

}  // namespace

bool attention_supported(int64_t T, int64_t dh) { return dh == kDH && (T == 64 || T == 128); }

void attention_fwd(const AttnDesc& a, hipStream_t st) {
  const int blocks = a.B * a.H * (a.T / kQB);
  if (blocks <= 0) return;
  if (a.T == 128) k_attn_fwd<128><<<blocks, kNT, 0, st>>>(a);
  else k_attn_fwd<64><<<blocks, kNT, 0, st>>>(a);
}

}  // namespace tgk
