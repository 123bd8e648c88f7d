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

template <int MODE, int BM, int BN>
__global__ __launch_bounds__(kCT) void k_conv_gemm(ConvGemmArgs c) {
  constexpr int WGM = BM >= 64 ? 2 : 1, WGN = 4 / WGM;   // wave grid
  constexpr int WM = BM / WGM, WN = BN / WGN;            // wave tile
  constexpr int TM = WM / 32, TN = WN / 32;
  static_assert(TM >= 1 && TN >= 1 && WM % 32 == 0 && WN % 32 == 0, "bad conv tile");
  constexpr bool BKF = MODE == CV_WGRAD;
  using SA = Stage<BM, true>;
  using SB = Stage<BN, BKF>;
  __shared__ __attribute__((aligned(16))) float As[2][SA::SIZE];
  __shared__ __attribute__((aligned(16))) float Bs[2][SB::SIZE];

  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
  // Tiles of one z (one image and group, or one split) are numbered contiguously per XCD.
  const uint32_t nblk = gridDim.x;
  uint32_t bid = blockIdx.x;
  if (nblk % kXcds == 0) bid = (bid % kXcds) * (nblk / kXcds) + bid / kXcds;
  const int tn = bid % c.tiles_n;
  const uint32_t rest = bid / c.tiles_n;
  const int tm = rest % c.tiles_m;
  const int zs = rest / c.tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const int z = MODE == CV_WGRAD ? zs / c.splits : zs;
  const int split = MODE == CV_WGRAD ? zs % c.splits : 0;
  const int kbeg = split * c.k_per_split;
  const int kend = min(c.K, kbeg + c.k_per_split);

  SA sa;
  SB sb;
  auto load = [&](int k0) {
#pragma unroll
    for (int e = 0; e < SA::Q; ++e) {
      int rr, kk;
      SA::coords(tid + e * kCT, rr, kk);
      sa.q[e] = a_elems<MODE>(c, z, m0 + rr, k0 + kk, kend);
    }
#pragma unroll
    for (int e = 0; e < SB::Q; ++e) {
      int rr, kk;
      SB::coords(tid + e * kCT, rr, kk);
      if (BKF) sb.q[e] = b_elems_k(c, z, n0 + rr, k0 + kk, kend);
      else sb.q[e] = b_elems_n<MODE>(c, z, n0 + rr, k0 + kk, kend);
    }
  };

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
    load(kbeg);
    sa.store(As[0], tid);
    sb.store(Bs[0], tid);
  }
  __syncthreads();
  for (int st = 0; st < nst; ++st) {
    const int cur = st & 1;
    const bool more = st + 1 < nst;
    if (more) load(kbeg + (st + 1) * kCBK);
    const float* Ac = As[cur];
    const float* Bc = Bs[cur];
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

  // Register r of lane l holds row (r/4)*8 + (l/32)*4 + r%4, column l%32.
  float* O;
  int64_t row_stride;
  if (MODE == CV_FWD) {
    const int b = fdiv(z, c.dG), g = z - b * c.G;
    O = c.out + ((int64_t)b * c.Cout + g * c.CoutPG) * c.N;
    row_stride = c.N;
  } else if (MODE == CV_DGRAD) {
    const int b = fdiv(z, c.dG), g = z - b * c.G;
    O = c.out + ((int64_t)b * c.Cin + g * c.CinPG) * c.N;
    row_stride = c.N;
  } else {
    O = c.splits > 1 ? c.work + ((int64_t)split * c.G + z) * c.M * c.N : c.out + (int64_t)z * c.M * c.N;
    row_stride = c.N;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int gn = n0 + wn0 + j * 32 + lrow;
      if (gn >= c.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gm = m0 + wm0 + i * 32 + (r / 4) * 8 + h * 4 + (r % 4);
        if (gm < c.M) O[gm * row_stride + gn] = acc[i][j][r];
      }
    }
}

// dW = sum of the split partials, in split order.
__global__ void k_conv_wgrad_reduce(const float* __restrict__ work, int splits, int64_t per_split,
                                    float* __restrict__ dw) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < per_split; i += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.0f;
    for (int sp = 0; sp < splits; ++sp) s += work[sp * per_split + i];
    dw[i] = s;
  }
}

template <int MODE>
void launch_mode(const ConvPlan& p, const ConvGemmArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)p.blocks);
  if (p.bm == 32) k_conv_gemm<MODE, 32, 128><<<grid, kCT, 0, st>>>(a);
  else if (p.bn == 128) k_conv_gemm<MODE, 64, 128><<<grid, kCT, 0, st>>>(a);
  else k_conv_gemm<MODE, 64, 64><<<grid, kCT, 0, st>>>(a);
}

}  // namespace

bool conv_gemm_ok(const ConvDesc& d) { return conv_ok(d); }

int64_t conv_gemm_workspace_bytes(const ConvDesc& d) {
  const ConvPlan p = conv_plan(CV_WGRAD, d);
  if (p.splits <= 1) return 0;
  return (int64_t)p.splits * d.G * (d.Cout / d.G) * d.CinPG * d.kH * d.kW * 4;
}

void conv2d_gemm(const float* x, const float* w, float* y, const ConvDesc& d, hipStream_t st) {
  const ConvPlan p = conv_plan(CV_FWD, d);
  ConvGemmArgs a = make_args(d, p);
  a.x = x; a.w = w; a.out = y;
  if (p.blocks > 0) launch_mode<CV_FWD>(p, a, st);
}

void conv2d_input_grad_gemm(const float* w, const float* dy, float* dx, const ConvDesc& d, hipStream_t st) {
  const ConvPlan p = conv_plan(CV_DGRAD, d);
  ConvGemmArgs a = make_args(d, p);
  a.w = w; a.dy = dy; a.out = dx;
  if (p.blocks > 0) launch_mode<CV_DGRAD>(p, a, st);
}

void conv2d_weight_grad_gemm(const float* x, const float* dy, float* dw, const ConvDesc& d, float* work,
                             hipStream_t st) {
  const ConvPlan p = conv_plan(CV_WGRAD, d);
  ConvGemmArgs a = make_args(d, p);
  a.x = x; a.dy = dy; a.out = dw; a.work = work;
  if (p.blocks <= 0) return;
  if (p.splits > 1 && !work) throw std::runtime_error("conv2d_weight_grad: missing workspace");
  launch_mode<CV_WGRAD>(p, a, st);
  if (p.splits > 1) {
    const int64_t per = (int64_t)a.G * a.M * a.N;
    const int64_t nb = std::min<int64_t>((per + 255) / 256, 4096);
    k_conv_wgrad_reduce<<<(int)nb, 256, 0, st>>>(work, p.splits, per, dw);
  }
}

}  // namespace tgk
