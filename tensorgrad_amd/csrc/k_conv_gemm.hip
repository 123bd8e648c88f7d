// Implicit-GEMM convolution (NCHW, f32) on the gfx950 matrix cores
// (v_mfma_f32_32x32x2_f32). Nothing is materialised: each operand tile is gathered from
// the activations with the convolution's index map while it is staged into LDS.
//
// Per image b and group g (z = b * G + g), the three IR kinds are GEMMs
//   conv2d            Y[co][p]   = sum_k W[co][k]        * X^[k][p]    k = (cl, kh, kw), p = (ho, wo)
//   conv2d_input_grad dX[cl][q]  = sum_k W^T[cl][k]      * dY^[k][q]   k = (col, kh, kw), q = (hi, wi)
//   conv2d_weight_grad dW[co][n] = sum_k dY[co][k]       * X~[k][n]    k = (b, ho, wo), n = (cl, kh, kw)
// with X^[k][p] = x[b, g*CinPG+cl, ho*sH+kh-pH, wo*sW+kw-pW] (zero outside the image),
// dY^[k][q] = dy[b, g*CoutPG+col, ho, wo] for the (ho, wo) with ho*sH+kh-pH = hi and
// wo*sW+kw-pW = wi (zero when there is none), and X~ the same gather as X^ with the roles
// of k and n exchanged. The weight gradient reduces over the whole batch, so its k range
// is split across blocks (deterministic: each split writes its own partial tile, a second
// kernel adds the partials in split order).
//
// The tile machinery follows k_gemm (k_gemm.hip): 256 threads, 32 x 32 MFMA wave tiles,
// k-permuted fragments (lane half h takes k = 4h .. 4h+3 of each group of 8), one fresh
// accumulator per BK-k stage added to the running sum (blocked summation), double-buffered
// LDS stages filled from registers prefetched during the previous stage's products.
// A (the weight or dY operand) is staged k-contiguous, [row][BK + 4]; B is staged in the
// direction its gather is contiguous: output positions (conv2d, input grad: consecutive
// wo / wi) as [k][BN + 8], or k (weight grad: consecutive wo) as [n][BK + 4]. Every
// index is 32-bit (the host checks that every tensor has fewer than 2^31 elements) and
// divisions by the geometry use precomputed multiplicative inverses (FastDiv).
#include "conv_gemm_dev.h"

#include <algorithm>
#include <stdexcept>

namespace tgk {
namespace {

using namespace gd;
using namespace cg;


// One operand's ROWS x BK stage in registers, as Tile in k_gemm.hip.
template <int ROWS, bool KFAST>
struct Stage {
  static constexpr int LD = KFAST ? kCBK + 4 : ROWS + 8;
  static constexpr int SIZE = KFAST ? ROWS * LD : kCBK * LD;
  static constexpr int Q = ROWS * kCBK / (4 * kCT);
  static_assert(Q >= 1, "tile too small for the block");
  f32x4 q[Q];

  __device__ __forceinline__ static void coords(int idx, int& rr, int& kk) {
    if (KFAST) { rr = idx / (kCBK / 4); kk = (idx % (kCBK / 4)) * 4; }
    else { rr = (idx % (ROWS / 4)) * 4; kk = idx / (ROWS / 4); }
  }
  __device__ __forceinline__ void store(float* L, int tid) const {
#pragma unroll
    for (int e = 0; e < Q; ++e) {
      int rr, kk;
      coords(tid + e * kCT, rr, kk);
      if (KFAST) *reinterpret_cast<f32x4*>(L + rr * LD + kk) = q[e];
      else *reinterpret_cast<f32x4*>(L + kk * LD + rr) = q[e];
    }
  }
  __device__ __forceinline__ static f32x4 frag(const float* L, int row, int kb) {
    if (KFAST) return *reinterpret_cast<const f32x4*>(L + row * LD + kb);
    f32x4 v;
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = L[(kb + u) * LD + row];
    return v;
  }
};

// Pipeline: two register sets of staged loads, so the global loads of stage s + 2 are in
// flight while stage s is multiplied and stage s + 1 waits in registers for its LDS slot.
template <int MODE, bool FAST, int BM, int BN, int F>
__global__ __launch_bounds__(kCT) void k_conv_gemm(ConvGemmArgs c) {
  constexpr int WGM = BM >= 64 ? 2 : 1, WGN = 4 / WGM;   // wave grid
  constexpr int WM = BM / WGM, WN = BN / WGN;            // wave tile
  constexpr int TM = WM / 32, TN = WN / 32;
  static_assert(TM >= 1 && TN >= 1 && WM % 32 == 0 && WN % 32 == 0, "bad conv tile");
  using L = ConvLoader<MODE, FAST, BM, BN, F>;
  using SA = Stage<BM, true>;
  using SB = Stage<BN, L::BKF>;
  static_assert(SA::Q == L::QA && SB::Q == L::QB, "stage / loader mismatch");
  constexpr bool TAB = (F & F_TAB) != 0;
  __shared__ __attribute__((aligned(16))) float As[2][SA::SIZE];
  __shared__ __attribute__((aligned(16))) float Bs[2][SB::SIZE];
  __shared__ uint32_t ktab[TAB ? 2 * kTab : 2];

  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
  L ld;
  ld.init(c, block_pos<BM, BN>(c, blockIdx.x, gridDim.x, MODE), tid);
  const int kbeg = ld.bp.kbeg, kend = ld.bp.kend;
  if (TAB) {
    for (int k = tid; k < c.K; k += kCT) k_term(c, MODE, k, ktab[2 * k], ktab[2 * k + 1]);
    __syncthreads();
  }

  SA sa[2];
  SB sb[2];
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int lrow = lane % 32, h = lane / 32;
  const int nst = kbeg < kend ? (kend - kbeg + kCBK - 1) / kCBK : 0;
  if (nst > 0) {
    ld.load(c, kbeg, sa[0].q, sb[0].q, ktab);
    if (nst > 1) ld.load(c, kbeg + kCBK, sa[1].q, sb[1].q, ktab);
    sa[0].store(As[0], tid);
    sb[0].store(Bs[0], tid);
  }
  __syncthreads();
  for (int st = 0; st < nst; ++st) {
    const int cur = st & 1;
    // registers of stage st were stored at the previous iteration: refill them with st + 2
    if (st + 2 < nst) {
      if (cur == 0) ld.load(c, kbeg + (st + 2) * kCBK, sa[0].q, sb[0].q, ktab);
      else ld.load(c, kbeg + (st + 2) * kCBK, sa[1].q, sb[1].q, ktab);
    }
    const float* Ac = As[cur];
    const float* Bc = Bs[cur];
    // Blocked accumulation: a fresh partial sum per stage, added to the running total.
    f32x16 part[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) part[i][j][r] = 0.0f;
#pragma unroll
    for (int grp = 0; grp < kCBK / 8; ++grp) {
      const int kb = grp * 8 + h * 4;
      f32x4 av[TM], bv[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) av[i] = SA::frag(Ac, wm0 + i * 32 + lrow, kb);
#pragma unroll
      for (int j = 0; j < TN; ++j) bv[j] = SB::frag(Bc, wn0 + j * 32 + lrow, kb);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            part[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][jj], bv[j][jj], part[i][j], 0, 0, 0);
    }
    if (st + 1 < nst) {
      if (cur == 0) { sa[1].store(As[1], tid); sb[1].store(Bs[1], tid); }
      else { sa[0].store(As[0], tid); sb[0].store(Bs[0], tid); }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] += part[i][j];
    __syncthreads();
  }

  // Register r of lane l holds row (r/4)*8 + (l/32)*4 + r%4, column l%32.
  float* O = (MODE == CV_WGRAD && c.splits > 1) ? c.work : c.out;
  const int64_t rs = ld.out_rs(c);
  if (MODE != CV_WGRAD && c.epi != kConvEpiNone) {
    // The layer's pointwise step at the store (one group, G = 1: channel gm). Every bias /
    // mask value of the wavefront's outputs is loaded first (clamped in range): loaded
    // between the stores, each would wait for the stores before it.
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int gn = min(ld.bp.n0 + wn0 + j * 32 + lrow, c.N - 1);
      const int64_t cofs = ld.out_col(c, gn);
      float e[TM][16];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int gm = min(ld.bp.m0 + wm0 + i * 32 + (r / 4) * 8 + h * 4 + (r % 4), c.M - 1);
          e[i][r] = c.epi == kConvEpiBiasRelu ? c.ebias[gm] : c.emask[cofs + gm * rs];
        }
      if (ld.bp.n0 + wn0 + j * 32 + lrow >= c.N) continue;
      float* col = O + cofs;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int gm = ld.bp.m0 + wm0 + i * 32 + (r / 4) * 8 + h * 4 + (r % 4);
          if (gm >= c.M) continue;
          float v = acc[i][j][r];
          if (c.epi == kConvEpiBiasRelu) {
            const float a = v + e[i][r];
            v = a != a ? __uint_as_float(0x7fc00000u) : (a > 0.0f ? a : 0.0f);
          } else {
            v = e[i][r] > 0.0f ? v : 0.0f;
          }
          col[gm * rs] = v;
        }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int gn = ld.bp.n0 + wn0 + j * 32 + lrow;
    if (gn >= c.N) continue;
    float* col = O + ld.out_col(c, gn);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gm = ld.bp.m0 + wm0 + i * 32 + (r / 4) * 8 + h * 4 + (r % 4);
        if (gm < c.M) col[gm * rs] = acc[i][j][r];
      }
  }
}

// dW = sum of the split partials, deterministic. Many outputs: a block of four wavefronts
// takes 64 consecutive outputs (coalesced), wavefront w adds splits w, w + 4, ... in order
// (8 loads in flight, clamped to split 0 past the end), and the four sums are added in
// order through LDS. Few outputs and many splits (small weights reducing over a large
// batch): one wavefront per output, lane l adding splits l, l + 64, ... in order, then a
// fixed butterfly across the lanes.
__global__ __launch_bounds__(256) void k_conv_wgrad_reduce(const float* __restrict__ work, int splits,
                                                           int64_t per_split, float* __restrict__ dw) {
  __shared__ float ws[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t i = (int64_t)blockIdx.x * 64 + lane;
  const int64_t ii = i < per_split ? i : per_split - 1;
  float s = 0.0f;
  for (int sp0 = w; sp0 < splits; sp0 += 4 * 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int sp = sp0 + 4 * u;
      v[u] = work[(int64_t)(sp < splits ? sp : 0) * per_split + ii];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (sp0 + 4 * u < splits) s += v[u];
  }
  ws[w][lane] = s;
  __syncthreads();
  if (w == 0 && i < per_split) dw[i] = ((ws[0][lane] + ws[1][lane]) + ws[2][lane]) + ws[3][lane];
}

__global__ __launch_bounds__(256) void k_conv_wgrad_reduce_wave(const float* __restrict__ work, int splits,
                                                                int64_t per_split, float* __restrict__ dw) {
  const int lane = threadIdx.x % 64;
  const int64_t i = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;   // one output per wavefront
  if (i >= per_split) return;                                      // uniform across the wavefront
  float s = 0.0f;
  for (int sp = lane; sp < splits; sp += 64) s += work[sp * per_split + i];
  s = wave_allsum(s);
  if (lane == 0) dw[i] = s;
}

// ---- convolutions with few taps ------------------------------------------------------------
// A first layer over 1-3 channel images has CinPG * kH * kW <= 16 taps per output: as a
// GEMM its forward has K <= 16 and its weight gradient N <= 16, so most of every 32-wide
// MFMA stage or tile would multiply padding. Both run on the vector ALU instead (f32 FMAs,
// GEMM tolerance like the MFMA path).
constexpr int kSmallTaps = 16;
constexpr int kSmallCo = 4;      // output channels per weight-gradient block
constexpr int kSmallW = 2048;    // forward: a group's weights staged in LDS, CoutPG * kSmallTaps floats

// Tap q = (cl, kh, kw) of an output position: its row and column shift and its channel
// plane offset, decoded once per thread.
struct SmallTaps {
  int dh[kSmallTaps], dw[kSmallTaps];
  uint32_t off[kSmallTaps];
  __device__ __forceinline__ void init(const ConvGemmArgs& c) {
#pragma unroll
    for (int q = 0; q < kSmallTaps; ++q) {
      const int qq = q < c.K ? q : 0;
      const int cl = fdiv(qq, c.dKHW), r = qq - cl * c.kH * c.kW;
      const int kh = fdiv(r, c.dKW), kw = r - kh * c.kW;
      dh[q] = kh - c.pH;
      dw[q] = kw - c.pW;
      off[q] = (uint32_t)(cl * c.H * c.W);
    }
  }
  // The taps of output position (ho, wo) of image plane base `base` (x's (b, g * CinPG)
  // offset), zero outside the image: raw buffer loads, masked ones at an out-of-range
  // offset, so all of them are in flight together.
  __device__ __forceinline__ void gather(const ConvGemmArgs& c, const Src& sx, uint32_t base, int ho, int wo,
                                         float* xv) const {
#pragma unroll
    for (int q = 0; q < kSmallTaps; ++q) {
      const int hi = ho * c.sH + dh[q], wi = wo * c.sW + dw[q];
      const bool ok = q < c.K && inside(hi, c.H) && inside(wi, c.W);
      xv[q] = ldb(sx, boff(ok, base + off[q] + (uint32_t)(hi * c.W + wi)));
    }
  }
};

// Forward: block (image b, group g, 256 positions), one thread per position, every output
// channel of the group from the group's weights in LDS, each row padded with zeros to
// kSmallTaps (the masked taps are zero too), so the product loop has no branches and reads
// each row as four 128-bit broadcasts.
__global__ __launch_bounds__(256) void k_conv_small_fwd(const ConvGemmArgs c) {
  __shared__ __attribute__((aligned(16))) float ws[kSmallW];
  __shared__ float bs[kSmallW / kSmallTaps];   // the group's biases (kConvEpiBiasRelu)
  const int hw = c.Ho * c.Wo;
  const int nchunk = (hw + 255) / 256;
  const int z = blockIdx.x / nchunk, chunk = blockIdx.x - z * nchunk;
  const int b = z / c.G, g = z - b * c.G;
  for (int i = threadIdx.x; i < c.CoutPG * kSmallTaps; i += 256) {
    const int co = i / kSmallTaps, q = i - co * kSmallTaps;
    ws[i] = q < c.K ? c.w[(int64_t)(g * c.CoutPG + co) * c.K + q] : 0.0f;
  }
  if (c.epi == kConvEpiBiasRelu)
    for (int i = threadIdx.x; i < c.CoutPG; i += 256) bs[i] = c.ebias[g * c.CoutPG + i];
  SmallTaps tp;
  tp.init(c);
  __syncthreads();
  const int p = chunk * 256 + threadIdx.x;
  if (p >= hw) return;
  const int ho = fdiv(p, c.dWo), wo = p - ho * c.Wo;
  const Src sx = make_src(c.x, (int64_t)c.B * c.Cin * c.H * c.W);
  float xv[kSmallTaps];
  tp.gather(c, sx, (uint32_t)((b * c.Cin + g * c.CinPG) * c.H * c.W), ho, wo, xv);
  float* y = c.out + (int64_t)(b * c.Cout + g * c.CoutPG) * hw + p;
  for (int co = 0; co < c.CoutPG; ++co) {
    const f32x4* wr = reinterpret_cast<const f32x4*>(ws + co * kSmallTaps);
    float s = 0.0f;
#pragma unroll
    for (int u = 0; u < kSmallTaps / 4; ++u) {
      const f32x4 w4 = wr[u];
#pragma unroll
      for (int e = 0; e < 4; ++e) s = fmaf(w4[e], xv[u * 4 + e], s);
    }
    if (c.epi == kConvEpiBiasRelu) {   // the bias from LDS
      const float a = s + bs[co];
      s = a != a ? __uint_as_float(0x7fc00000u) : (a > 0.0f ? a : 0.0f);
    }
    y[(int64_t)co * hw] = s;
  }
}

// Weight gradient: block (ipb consecutive images, group g, kSmallCo output channels) sums
// dy * tap over the images' positions (threads take positions t, t + 256, ... of each image
// in turn), then across the block in a fixed order: every thread stores its sums in LDS,
// four threads per sum add 64 threads' values each in thread order, and the four quarters
// are added in order, giving the image group's partial dW rows work[ig][g * CoutPG + co][q].
// The partials are added in image-group order. Several images per block spread the fixed
// cost of the block sum over more positions.
__global__ __launch_bounds__(256) void k_conv_small_wgrad(const ConvGemmArgs c) {
  constexpr int NV = kSmallCo * kSmallTaps;
  static_assert(NV * 4 == 256, "four threads per sum");
  __shared__ float red[256][NV + 1];
  const int hw = c.Ho * c.Wo;
  const int nch = (c.CoutPG + kSmallCo - 1) / kSmallCo;
  const int blk = blockIdx.x, cc = blk % nch, z = blk / nch;
  const int ig = z / c.G, g = z - ig * c.G;
  const int tid = threadIdx.x;
  SmallTaps tp;
  tp.init(c);
  const Src sx = make_src(c.x, (int64_t)c.B * c.Cin * c.H * c.W);
  const Src sdy = make_src(c.dy, (int64_t)c.B * c.Cout * hw);
  float acc[kSmallCo][kSmallTaps];
#pragma unroll
  for (int j = 0; j < kSmallCo; ++j)
#pragma unroll
    for (int q = 0; q < kSmallTaps; ++q) acc[j][q] = 0.0f;
  const int bend = min(c.B, (ig + 1) * c.ipb);
  for (int b = ig * c.ipb; b < bend; ++b) {
    const uint32_t xbase = (uint32_t)((b * c.Cin + g * c.CinPG) * c.H * c.W);
    const uint32_t dbase = (uint32_t)((b * c.Cout + g * c.CoutPG + cc * kSmallCo) * hw);
    for (int p = tid; p < hw; p += 256) {
      const int ho = fdiv(p, c.dWo), wo = p - ho * c.Wo;
      float xv[kSmallTaps], d[kSmallCo];
      tp.gather(c, sx, xbase, ho, wo, xv);
#pragma unroll
      for (int j = 0; j < kSmallCo; ++j)
        d[j] = ldb(sdy, boff(cc * kSmallCo + j < c.CoutPG, dbase + (uint32_t)(j * hw + p)));
#pragma unroll
      for (int j = 0; j < kSmallCo; ++j)
#pragma unroll
        for (int q = 0; q < kSmallTaps; ++q) acc[j][q] = fmaf(d[j], xv[q], acc[j][q]);
    }
  }
#pragma unroll
  for (int j = 0; j < kSmallCo; ++j)
#pragma unroll
    for (int q = 0; q < kSmallTaps; ++q) red[tid][j * kSmallTaps + q] = acc[j][q];
  __syncthreads();
  const int v = tid % NV, quarter = tid / NV;   // 256 threads = 4 quarters of the NV sums
  float s = 0.0f;
  for (int i = 0; i < 64; ++i) s += red[quarter * 64 + i][v];
  __syncthreads();
  red[quarter][v] = s;
  __syncthreads();
  if (tid < NV) {
    const int j = tid / kSmallTaps, q = tid % kSmallTaps, co = cc * kSmallCo + j;
    if (co < c.CoutPG && q < c.K) {
      const float t = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
      c.work[(int64_t)ig * c.G * c.CoutPG * c.K + (int64_t)(g * c.CoutPG + co) * c.K + q] = t;
    }
  }
}

// The few-taps weight gradient applies when its per-image partials fit the workspace.
bool small_wgrad_ok(const ConvDesc& d) {
  const int64_t taps = d.CinPG * d.kH * d.kW;
  return taps <= kSmallTaps && d.B * d.Cout * taps * 4 <= kConvWorkBytes;
}

template <int MODE, bool FAST, int F>
void launch_tile(const ConvPlan& p, const ConvGemmArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)p.blocks);
  if (p.bm == 32) klaunch(k_conv_gemm<MODE, FAST, 32, 128, F>, grid, kCT, 0, st, a);
  else if (p.bn == 64) klaunch(k_conv_gemm<MODE, FAST, 64, 64, F>, grid, kCT, 0, st, a);
  else klaunch(k_conv_gemm<MODE, FAST, 64, 128, F>, grid, kCT, 0, st, a);
}

// The loader variant (conv_flags) of a launch picks the instantiation.
template <int MODE>
void launch_mode(const ConvPlan& p, const ConvGemmArgs& a, bool fast, hipStream_t st) {
  const int f = conv_flags(a, MODE);
  if (MODE == CV_DGRAD && fast && (f & F_TAP)) return launch_tile<MODE, true, F_TAP>(p, a, st);
  if (MODE == CV_FWD && (f & F_TAP)) {
    if (f & F_PAD) launch_tile<MODE, true, F_TAP | F_PAD>(p, a, st);
    else launch_tile<MODE, true, F_TAP>(p, a, st);
    return;
  }
  if (MODE == CV_DGRAD) {
    if (!fast) launch_tile<MODE, false, 0>(p, a, st);
    else if (f & F_TAB) launch_tile<MODE, true, F_TAB>(p, a, st);
    else launch_tile<MODE, true, 0>(p, a, st);
    return;
  }
  const int fa = f & (F_AVEC | F_PAD);
  if (MODE == CV_FWD && (f & F_TAB)) {
    switch (fa) {
      case 0: launch_tile<MODE, true, F_TAB>(p, a, st); return;
      case F_AVEC: launch_tile<MODE, true, F_TAB | F_AVEC>(p, a, st); return;
      case F_PAD: launch_tile<MODE, true, F_TAB | F_PAD>(p, a, st); return;
      default: launch_tile<MODE, true, F_TAB | F_AVEC | F_PAD>(p, a, st); return;
    }
  }
  switch (fa) {
    case 0: launch_tile<MODE, true, 0>(p, a, st); return;
    case F_AVEC: launch_tile<MODE, true, F_AVEC>(p, a, st); return;
    case F_PAD: launch_tile<MODE, true, F_PAD>(p, a, st); return;
    default: launch_tile<MODE, true, F_AVEC | F_PAD>(p, a, st); return;
  }
}

}  // namespace

bool conv_gemm_ok(const ConvDesc& d) { return conv_ok(d); }

int64_t conv_gemm_workspace_bytes(const ConvDesc& d) {
  if (small_wgrad_ok(d)) return d.B * d.Cout * d.CinPG * d.kH * d.kW * 4;
  const ConvPlan p = conv_plan(CV_WGRAD, d);
  if (p.splits <= 1) return 0;
  return (int64_t)p.splits * d.G * (d.Cout / d.G) * d.CinPG * d.kH * d.kW * 4;
}

void conv2d_gemm(const float* x, const float* w, float* y, const ConvDesc& d, hipStream_t st, const float* bias) {
  const ConvPlan p = conv_plan(CV_FWD, d);
  ConvGemmArgs a = make_args(d, p);
  a.x = x; a.w = w; a.out = y;
  if (bias) {
    if (d.G != 1) throw std::runtime_error("conv2d: a bias epilogue needs one group");
    a.epi = kConvEpiBiasRelu;
    a.ebias = bias;
  }
  a.avec = a.avec && ((uintptr_t)w & 15) == 0;
  if (d.CinPG * d.kH * d.kW <= kSmallTaps && (d.Cout / d.G) * kSmallTaps <= kSmallW) {
    // the K taps of a row of W are contiguous: W[co][cl][kh][kw] = w[co * K + q]
    const int64_t n = d.B * d.G * ((d.Ho * d.Wo + 255) / 256);
    if (n > 0) klaunch(k_conv_small_fwd, (unsigned)n, 256, 0, st, a);
    return;
  }
  if (p.blocks > 0) launch_mode<CV_FWD>(p, a, true, st);
}

void conv2d_input_grad_gemm(const float* w, const float* dy, float* dx, const ConvDesc& d, hipStream_t st,
                            const float* mask) {
  const ConvPlan p = conv_plan(CV_DGRAD, d);
  ConvGemmArgs a = make_args(d, p);
  a.w = w; a.dy = dy; a.out = dx;
  if (mask) {
    a.epi = kConvEpiReluMask;
    a.emask = mask;
  }
  if (p.blocks > 0) launch_mode<CV_DGRAD>(p, a, d.sH == 1 && d.sW == 1, st);
}

void conv2d_weight_grad_gemm(const float* x, const float* dy, float* dw, const ConvDesc& d, float* work,
                             hipStream_t st) {
  const ConvPlan p = conv_plan(CV_WGRAD, d);
  ConvGemmArgs a = make_args(d, p);
  a.x = x; a.dy = dy; a.out = dw; a.work = work;
  a.avec = a.avec && ((uintptr_t)dy & 15) == 0;
  if (small_wgrad_ok(d)) {
    if (!work) throw std::runtime_error("conv2d_weight_grad: missing workspace");
    if (d.B <= 0 || d.Cout <= 0) return;
    ConvGemmArgs sa = a;   // K: the taps per output (the GEMM view's N)
    sa.K = (int)(d.CinPG * d.kH * d.kW);
    const int64_t per = d.Cout * sa.K;
    const int64_t nch = (a.CoutPG + kSmallCo - 1) / kSmallCo;
    // images per block: about two blocks per CU (the block sum's LDS admits two)
    sa.ipb = (int)std::max<int64_t>(1, d.B * d.G * nch / 512);
    const int64_t ngroups = (d.B + sa.ipb - 1) / sa.ipb;
    klaunch(k_conv_small_wgrad, (unsigned)(ngroups * d.G * nch), 256, 0, st, sa);
    if (per < 16384 && ngroups > 16) {
      klaunch(k_conv_wgrad_reduce_wave, (unsigned)((per + 3) / 4), 256, 0, st, work, (int)ngroups, per, dw);
    } else {
      klaunch(k_conv_wgrad_reduce, (unsigned)((per + 63) / 64), 256, 0, st, work, (int)ngroups, per, dw);
    }
    return;
  }
  if (p.blocks <= 0) return;
  if (p.splits > 1 && !work) throw std::runtime_error("conv2d_weight_grad: missing workspace");
  launch_mode<CV_WGRAD>(p, a, true, st);
  if (p.splits > 1) {
    const int64_t per = (int64_t)a.G * a.M * a.N;
    if (per < 16384 && p.splits > 16) {
      klaunch(k_conv_wgrad_reduce_wave, (unsigned)((per + 3) / 4), 256, 0, st, work, p.splits, per, dw);
    } else {
      klaunch(k_conv_wgrad_reduce, (unsigned)((per + 63) / 64), 256, 0, st, work, p.splits, per, dw);
    }
  }
}

}  // namespace tgk
