// Index maps and launch plan of the implicit-GEMM convolutions (k_conv_gemm.hip), kept
// in a header of host + device functions so that the same code can be exercised on the CPU.
#pragma once
#include <algorithm>
#include <cstdint>

#include "kernels.h"

namespace tgk {
namespace cg {

using gd::f32x4;

#define CG_HD __host__ __device__ __forceinline__

constexpr int kCT = 256;
constexpr int kCBK = 32;

enum { CV_FWD = 0, CV_DGRAD = 1, CV_WGRAD = 2 };

struct ConvGemmArgs {
  int B, Cin, H, W, Cout, CinPG, CoutPG, kH, kW, Ho, Wo, G, sH, sW, pH, pW;
  int M, N, K;                  // GEMM sizes per z
  int tiles_m, tiles_n, splits, k_per_split;
  FastDiv dKHW, dKW, dWo, dHoWo, dW, dG, dSH, dSW;
  const float* x;
  const float* w;
  const float* dy;
  float* out;                   // y / dx / dw
  float* work;                  // weight-gradient partials [split][G][M][N] (splits > 1)
};

// x / d for 0 <= x < 2^31 (FastDiv, kernels.h), on the host or the device.
CG_HD int fdiv(int x, const FastDiv& f) {
  return (int)((((uint32_t)(((uint64_t)(uint32_t)x * f.m) >> 32)) + (uint32_t)x) >> f.s);
}

// ---- operand A: k-contiguous rows ------------------------------------------------------
template <int MODE>
CG_HD f32x4 a_elems(const ConvGemmArgs& c, int z, int m, int k0, int kend) {
  f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
  if (m >= c.M) return v;
  if (MODE == CV_FWD) {
    const int g = z - fdiv(z, c.dG) * c.G;
    const float* row = c.w + (int64_t)(g * c.CoutPG + m) * c.K;
#pragma unroll
    for (int u = 0; u < 4; ++u) if (k0 + u < kend) v[u] = row[k0 + u];
  } else if (MODE == CV_DGRAD) {
    const int g = z - fdiv(z, c.dG) * c.G;
    const int khw = c.kH * c.kW;
    int col = fdiv(k0, c.dKHW), r = k0 - col * khw;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (k0 + u < kend) v[u] = c.w[((int64_t)(g * c.CoutPG + col) * c.CinPG + m) * khw + r];
      if (++r == khw) { r = 0; ++col; }
    }
  } else {   // CV_WGRAD: dY[co][(b, p)]
    const int hw = c.Ho * c.Wo;
    int b = fdiv(k0, c.dHoWo), p = k0 - b * hw;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (k0 + u < kend) v[u] = c.dy[((int64_t)b * c.Cout + z * c.CoutPG + m) * hw + p];
      if (++p == hw) { p = 0; ++b; }
    }
  }
  return v;
}

// ---- operand B, staged by output position (conv2d, input gradient): 4 consecutive n -----
template <int MODE>
CG_HD f32x4 b_elems_n(const ConvGemmArgs& c, int z, int n0, int k, int kend) {
  f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
  if (k >= kend || n0 >= c.N) return v;
  const int b = fdiv(z, c.dG), g = z - b * c.G;
  const int khw = c.kH * c.kW;
  const int kc = fdiv(k, c.dKHW), r = k - kc * khw;
  const int kh = fdiv(r, c.dKW), kw = r - kh * c.kW;
  if (MODE == CV_FWD) {
    const float* plane = c.x + ((int64_t)b * c.Cin + g * c.CinPG + kc) * c.H * c.W;
    int ho = fdiv(n0, c.dWo), wo = n0 - ho * c.Wo;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int hi = ho * c.sH + kh - c.pH, wi = wo * c.sW + kw - c.pW;
      if (n0 + u < c.N && hi >= 0 && hi < c.H && wi >= 0 && wi < c.W) v[u] = plane[hi * c.W + wi];
      if (++wo == c.Wo) { wo = 0; ++ho; }
    }
  } else {   // CV_DGRAD
    const float* plane = c.dy + ((int64_t)b * c.Cout + g * c.CoutPG + kc) * c.Ho * c.Wo;
    int hi = fdiv(n0, c.dW), wi = n0 - hi * c.W;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int nh = hi + c.pH - kh, nw = wi + c.pW - kw;
      if (n0 + u < c.N && nh >= 0 && nw >= 0) {
        const int ho = fdiv(nh, c.dSH), wo = fdiv(nw, c.dSW);
        if (ho * c.sH == nh && wo * c.sW == nw && ho < c.Ho && wo < c.Wo) v[u] = plane[ho * c.Wo + wo];
      }
      if (++wi == c.W) { wi = 0; ++hi; }
    }
  }
  return v;
}

// ---- operand B of the weight gradient, staged by k: 4 consecutive (b, ho, wo) ------------
CG_HD f32x4 b_elems_k(const ConvGemmArgs& c, int g, int n, int k0, int kend) {
  f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
  if (n >= c.N) return v;
  const int khw = c.kH * c.kW;
  const int cl = fdiv(n, c.dKHW), r = n - cl * khw;
  const int kh = fdiv(r, c.dKW), kw = r - kh * c.kW;
  const int hw = c.Ho * c.Wo;
  int b = fdiv(k0, c.dHoWo), p = k0 - b * hw;
  int ho = fdiv(p, c.dWo), wo = p - ho * c.Wo;
  const int64_t plane = (int64_t)c.H * c.W;
  const float* base = c.x + (int64_t)(g * c.CinPG + cl) * plane;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int hi = ho * c.sH + kh - c.pH, wi = wo * c.sW + kw - c.pW;
    if (k0 + u < kend && hi >= 0 && hi < c.H && wi >= 0 && wi < c.W)
      v[u] = base[(int64_t)b * c.Cin * plane + hi * c.W + wi];
    if (++wo == c.Wo) {
      wo = 0;
      if (++ho == c.Ho) { ho = 0; ++b; }
    }
  }
  return v;
}

struct ConvPlan { int mode, bm, bn, splits, k_per_split, tiles_m, tiles_n; int64_t blocks; };

inline ConvPlan conv_plan(int mode, const ConvDesc& d) {
  ConvPlan p{};
  p.mode = mode;
  const int64_t M = mode == CV_DGRAD ? d.CinPG : d.Cout / d.G;
  const int64_t N = mode == CV_FWD ? d.Ho * d.Wo : mode == CV_DGRAD ? d.H * d.W : d.CinPG * d.kH * d.kW;
  const int64_t K = mode == CV_FWD ? d.CinPG * d.kH * d.kW
                    : mode == CV_DGRAD ? (d.Cout / d.G) * d.kH * d.kW : d.B * d.Ho * d.Wo;
  const int64_t Z = mode == CV_WGRAD ? d.G : d.B * d.G;
  p.bm = M <= 32 ? 32 : 64;
  p.bn = p.bm == 32 ? 128 : (N >= 1024 ? 128 : 64);
  p.tiles_m = (int)((M + p.bm - 1) / p.bm);
  p.tiles_n = (int)((N + p.bn - 1) / p.bn);
  p.splits = 1;
  p.k_per_split = (int)K;
  if (mode == CV_WGRAD) {
    // Enough blocks to fill the chip twice over, each split at least 8 k stages, and the
    // partials within kConvWorkBytes.
    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n * Z;
    int64_t s = (512 + tiles - 1) / tiles;
    s = std::min<int64_t>(s, std::max<int64_t>(1, K / (8 * kCBK)));
    const int64_t per = Z * M * N * 4;
    s = std::min<int64_t>(s, std::max<int64_t>(1, kConvWorkBytes / per));
    if (s > 1) {
      int64_t kps = (K + s - 1) / s;
      kps = (kps + kCBK - 1) / kCBK * kCBK;
      s = (K + kps - 1) / kps;
      p.k_per_split = (int)kps;
    }
    p.splits = (int)s;
  }
  p.blocks = (int64_t)p.tiles_m * p.tiles_n * Z * p.splits;
  return p;
}

inline ConvGemmArgs make_args(const ConvDesc& d, const ConvPlan& p) {
  ConvGemmArgs a{};
  a.B = (int)d.B; a.Cin = (int)d.Cin; a.H = (int)d.H; a.W = (int)d.W; a.Cout = (int)d.Cout;
  a.CinPG = (int)d.CinPG; a.CoutPG = (int)(d.Cout / d.G); a.kH = (int)d.kH; a.kW = (int)d.kW;
  a.Ho = (int)d.Ho; a.Wo = (int)d.Wo; a.G = (int)d.G; a.sH = (int)d.sH; a.sW = (int)d.sW;
  a.pH = (int)d.pH; a.pW = (int)d.pW;
  if (p.mode == CV_FWD) { a.M = a.CoutPG; a.N = a.Ho * a.Wo; a.K = a.CinPG * a.kH * a.kW; }
  else if (p.mode == CV_DGRAD) { a.M = a.CinPG; a.N = a.H * a.W; a.K = a.CoutPG * a.kH * a.kW; }
  else { a.M = a.CoutPG; a.N = a.CinPG * a.kH * a.kW; a.K = a.B * a.Ho * a.Wo; }
  a.tiles_m = p.tiles_m; a.tiles_n = p.tiles_n; a.splits = p.splits; a.k_per_split = p.k_per_split;
  a.dKHW = make_fastdiv((uint32_t)(a.kH * a.kW));
  a.dKW = make_fastdiv((uint32_t)a.kW);
  a.dWo = make_fastdiv((uint32_t)a.Wo);
  a.dHoWo = make_fastdiv((uint32_t)(a.Ho * a.Wo));
  a.dW = make_fastdiv((uint32_t)a.W);
  a.dG = make_fastdiv((uint32_t)a.G);
  a.dSH = make_fastdiv((uint32_t)a.sH);
  a.dSW = make_fastdiv((uint32_t)a.sW);
  return a;
}


// Every tensor and every launch indexable in 32 bits, and a geometry the maps assume.
inline bool conv_ok(const ConvDesc& d) {
  const int64_t lim = (int64_t(1) << 31) - 1;
  if (d.B <= 0 || d.G <= 0 || d.Cout % d.G != 0 || d.sH <= 0 || d.sW <= 0 || d.Ho <= 0 || d.Wo <= 0 || d.kH <= 0 ||
      d.kW <= 0 || d.pH < 0 || d.pW < 0)
    return false;
  const int64_t big = std::max({d.B * d.Cin * d.H * d.W, d.B * d.Cout * d.Ho * d.Wo, d.Cout * d.CinPG * d.kH * d.kW,
                                d.H + d.pH + d.kH, d.W + d.pW + d.kW});
  if (big >= lim) return false;
  for (int mode : {CV_FWD, CV_DGRAD, CV_WGRAD})
    if (conv_plan(mode, d).blocks >= lim) return false;
  return true;
}

#undef CG_HD

}  // namespace cg
}  // namespace tgk
