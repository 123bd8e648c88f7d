// Index maps, per-thread operand loaders and launch plan of the implicit-GEMM
// convolutions (k_conv_gemm.hip). Host + device code, so that the exact loaders the
// kernel runs can also be exercised on the CPU.
//
// GEMM view, per group g (images are folded into the spatial dimension):
//   conv2d             Y[co][(b,p)]  = sum_{k=(cl,kh,kw)}  W[co][k] * x[b, cl, ho*sH+kh-pH, wo*sW+kw-pW]
//   conv2d_input_grad  dX[cl][(b,q)] = sum_{k=(col,kh,kw)} W[col][cl][kh,kw] * dy[b, col, ho, wo],
//                                      (ho, wo) with ho*sH+kh-pH = hi, wo*sW+kw-pW = wi
//   conv2d_weight_grad dW[co][n=(cl,kh,kw)] = sum_{k=(b,p)} dy[b, co, p] * x[b, cl, ho*sH+kh-pH, wo*sW+kw-pW]
// with p = (ho, wo), q = (hi, wi). Out-of-image taps read as zero.
//
// The gathers are separable: the element offset is (a term of the output position) + (a
// term of the reduction index), e.g. for conv2d x offset = [b*Cin*HW + ho*sH*W + wo*sW]
// + [cl*HW + (kh-pH)*W + (kw-pW)]. Each thread computes the terms of the output positions
// it loads once per block and the terms of its k values once per stage, so a stage costs
// one add and (with padding) two unsigned compares per element. Offsets are 32-bit
// (every tensor has fewer than 2^29 elements; sums of a non-negative position term and a
// possibly negative k term are taken modulo 2^32, which is exact for in-range results).
// The input gradient with a stride above 1 uses a slower per-element map (divisibility
// of hi + pH - kh by sH).
#pragma once
#include <algorithm>
#include <cstdint>

#include "kernels.h"

namespace tgk {
namespace cg {

using gd::f32x4;

#define CG_HD __host__ __device__ __forceinline__

constexpr int kCT = 256;    // threads per block
constexpr int kCBK = 32;    // k per LDS stage
constexpr int kTab = 1024;  // conv2d / input gradient: k terms kept in an LDS table when K <= kTab

enum { CV_FWD = 0, CV_DGRAD = 1, CV_WGRAD = 2 };
// Loader variants, chosen per launch (template flags, so the k loop has no runtime tests):
// F_AVEC: A rows are 16-byte aligned groups of 4 k (vector loads); F_TAB: the k terms come
// from the block's LDS table; F_PAD: some tap falls outside the image (bounds checks);
// F_TAP: conv2d or the stride-1 input gradient with a multiple of kCBK channels per group
// runs its reduction tap-major, k = tap * channels + channel, so every stage holds one tap
// and 32 channels: a thread finds its positions' offsets and in-image tests once per stage
// and each element costs one add (the GEMM's k order changes, its value does not).
enum { F_AVEC = 1, F_TAB = 2, F_PAD = 4, F_TAP = 8 };

struct ConvGemmArgs {
  int B, Cin, H, W, Cout, CinPG, CoutPG, kH, kW, Ho, Wo, G, sH, sW, pH, pW;
  int M, N, K;                  // GEMM sizes per group
  int tiles_m, tiles_n, splits, k_per_split;
  int pad;                      // some tap can fall outside the image: bounds checks needed
  int avec;                     // A rows are 16-byte aligned in groups of 4 k (vector loads)
  int ipb;                      // few-taps weight gradient: images per block
  FastDiv dKHW, dKW, dWo, dHoWo, dW, dHW, dSH, dSW;
  FastDiv dCpg;                 // F_TAP: channels per group of the reduction (CinPG / CoutPG)
  const float* x;
  const float* w;
  const float* dy;
  float* out;                   // y / dx / dw
  float* work;                  // weight-gradient partials [split][G][M][N] (splits > 1)
  // A pointwise group applied at the store: kConvEpiBiasRelu on the forward's
  // output channel ch, kConvEpiReluMask on the input gradient's element.
  int epi;
  const float* ebias;           // [Cout]
  const float* emask;           // laid out as the output
};

// kConvEpiBiasRelu: relu(v + bias[ch]) as the fused group computes it (f32 add; relu keeps
// NaN as the canonical NaN and maps -0 to +0). kConvEpiReluMask: relu_grad(mask, v) =
// mask > 0 ? v : +0, the mask at the output element's offset.
constexpr int kConvEpiNone = 0, kConvEpiBiasRelu = 1, kConvEpiReluMask = 2;

// x / d for 0 <= x < 2^31 (FastDiv, kernels.h), on the host or the device.
CG_HD int fdiv(int x, const FastDiv& f) {
  return (int)((((uint32_t)(((uint64_t)(uint32_t)x * f.m) >> 32)) + (uint32_t)x) >> f.s);
}

CG_HD bool inside(int a, int lim) { return (uint32_t)a < (uint32_t)lim; }

// An operand tensor read through the buffer unit (raw buffer loads: 32-bit byte offsets
// from a uniform base, and offsets at or past the tensor's size read as 0 without a
// memory access). Masked elements are loaded from offset kMasked, so the loads need no
// branches. Tensors have fewer than 2^29 elements, so kMasked lies past every tensor and
// is 16-byte aligned. The host build (used to exercise the loaders on the CPU) reads the
// array directly with the same rule.
constexpr uint32_t kMasked = 0x80000000u;
struct Src {
#if defined(__HIP_DEVICE_COMPILE__)
  __amdgpu_buffer_rsrc_t r;
#else
  const float* p;
  uint32_t bytes;
#endif
};
CG_HD Src make_src(const float* p, int64_t elems) {
  Src s;
#if defined(__HIP_DEVICE_COMPILE__)
  // word 3 = 0x00020000: 32-bit data format, the setting for untyped loads on gfx9 parts
  s.r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, (int)(elems * 4), 0x00020000);
#else
  s.p = p;
  s.bytes = (uint32_t)(elems * 4);
#endif
  return s;
}
CG_HD float ldb(const Src& s, uint32_t off) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(s.r, (int)off, 0, 0));
#else
  return off < s.bytes ? s.p[off >> 2] : 0.0f;
#endif
}
CG_HD f32x4 ldb4(const Src& s, uint32_t off) {   // off 16-byte aligned
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(s.r, (int)off, 0, 0));
#else
  f32x4 v;
  for (int u = 0; u < 4; ++u) v[u] = off + 4 * u < s.bytes ? s.p[(off >> 2) + u] : 0.0f;
  return v;
#endif
}
CG_HD uint32_t boff(bool ok, uint32_t idx) { return ok ? idx << 2 : kMasked; }

// k term of conv2d / the stride-1 input gradient for reduction index k: the offset term
// and the two spatial shifts packed as 16-bit halves (low: row shift, high: column shift).
CG_HD void k_term(const ConvGemmArgs& c, int mode, int k, uint32_t& off, uint32_t& shifts) {
  const int khw = c.kH * c.kW;
  const int kc = fdiv(k, c.dKHW), r = k - kc * khw;
  const int kh = fdiv(r, c.dKW), kw = r - kh * c.kW;
  int a, b;
  if (mode == CV_FWD) {
    a = kh - c.pH;
    b = kw - c.pW;
    off = (uint32_t)(kc * c.H * c.W) + (uint32_t)(a * c.W + b);
  } else {
    a = kh;
    b = kw;
    off = (uint32_t)(kc * c.Ho * c.Wo) - (uint32_t)(kh * c.Wo + kw);
  }
  shifts = ((uint32_t)a & 0xFFFFu) | ((uint32_t)b << 16);
}
CG_HD int shift_lo(uint32_t s) { return (int)(int16_t)(s & 0xFFFFu); }
CG_HD int shift_hi(uint32_t s) { return (int)(int16_t)(s >> 16); }

// Block position in the launch grid: output tile (tm, tn), group z and k split.
struct BlockPos {
  int m0, n0, z, split, kbeg, kend;
};

template <int BM, int BN>
CG_HD BlockPos block_pos(const ConvGemmArgs& c, uint32_t blk, uint32_t nblk, int mode) {
  // Tiles are numbered so each XCD (the chip's 8 L2 domains take blocks round robin)
  // receives a contiguous run, n fastest.
  uint32_t bid = blk;
  if (nblk % gd::kXcds == 0) bid = (bid % gd::kXcds) * (nblk / gd::kXcds) + bid / gd::kXcds;
  BlockPos p;
  const int tn = bid % c.tiles_n;
  const uint32_t rest = bid / c.tiles_n;
  const int tm = rest % c.tiles_m;
  const int zs = rest / c.tiles_m;
  p.m0 = tm * BM;
  p.n0 = tn * BN;
  p.z = mode == CV_WGRAD ? zs / c.splits : zs;
  p.split = mode == CV_WGRAD ? zs % c.splits : 0;
  p.kbeg = p.split * c.k_per_split;
  p.kend = std::min(c.K, p.kbeg + c.k_per_split);
  return p;
}

// Register-staged coordinates of element group `e` of thread `tid` (as k_gemm's Tile):
// k-contiguous operands take 4 consecutive k of one row, row-contiguous ones 4
// consecutive rows at one k.
template <int ROWS, bool KFAST, int E>
CG_HD void stage_coords(int tid, int& rr, int& kk) {
  const int idx = tid + E * kCT;
  if (KFAST) { rr = idx / (kCBK / 4); kk = (idx % (kCBK / 4)) * 4; }
  else { rr = (idx % (ROWS / 4)) * 4; kk = idx / (ROWS / 4); }
}

// Per-thread loader of one block's operand stages. MODE selects the convolution kind;
// FAST = the separable maps (conv2d always, the input gradient at stride 1, the weight
// gradient always).
template <int MODE, bool FAST, int BM, int BN, int F>
struct ConvLoader {
  static constexpr bool BKF = MODE == CV_WGRAD;          // B staged k-contiguous
  static constexpr int QA = BM * kCBK / (4 * kCT);
  static constexpr int QB = BN * kCBK / (4 * kCT);
  BlockPos bp;
  int tid;
  Src sx, sw, sdy;  // x, w, dy
  // row-contiguous B (conv2d, input gradient): the thread's 4 output positions
  uint32_t nb[4];   // position term of the offset
  int ph[4], pw[4]; // spatial coordinates the k term's (dh, dw) is added to
  int nvalid;       // bit u: position u exists
  // k-contiguous B (weight gradient): the thread's output columns n, one per group
  uint32_t wnoff[QB > 0 ? QB : 1];
  int wdh[QB > 0 ? QB : 1], wdw[QB > 0 ? QB : 1];
  int wnvalid;      // bit e: column of group e exists

  CG_HD void init(const ConvGemmArgs& c, const BlockPos& p, int t) {
    bp = p;
    tid = t;
    sx = make_src(c.x, (int64_t)c.B * c.Cin * c.H * c.W);
    sw = make_src(c.w, (int64_t)c.Cout * c.CinPG * c.kH * c.kW);
    sdy = make_src(c.dy, (int64_t)c.B * c.Cout * c.Ho * c.Wo);
    nvalid = 0;
    wnvalid = 0;
    if (!BKF) {
      int rr, kk;
      stage_coords<BN, false, 0>(tid, rr, kk);   // every group of a thread has the same rows
      const int n0 = p.n0 + rr;
      const int g = p.z;
      if (MODE == CV_FWD) {
        const int hw = c.Ho * c.Wo;
        int b = n0 < c.N ? fdiv(n0, c.dHoWo) : 0;
        int q = n0 - b * hw;
        int ho = fdiv(q, c.dWo), wo = q - ho * c.Wo;
        for (int u = 0; u < 4; ++u) {
          if (n0 + u < c.N) {
            nvalid |= 1 << u;
            nb[u] = (uint32_t)(((b * c.Cin + g * c.CinPG) * c.H + ho * c.sH) * c.W + wo * c.sW);
            ph[u] = ho * c.sH;
            pw[u] = wo * c.sW;
          } else {
            nb[u] = 0; ph[u] = 0; pw[u] = 0;
          }
          if (++wo == c.Wo) { wo = 0; if (++ho == c.Ho) { ho = 0; ++b; } }
        }
      } else {   // CV_DGRAD: positions (b, hi, wi) of dX
        const int hw = c.H * c.W;
        int b = n0 < c.N ? fdiv(n0, c.dHW) : 0;
        int q = n0 - b * hw;
        int hi = fdiv(q, c.dW), wi = q - hi * c.W;
        for (int u = 0; u < 4; ++u) {
          if (n0 + u < c.N) {
            nvalid |= 1 << u;
            // stride 1: ho = hi + pH - kh, wo = wi + pW - kw
            nb[u] = (uint32_t)(((b * c.Cout + g * c.CoutPG) * c.Ho + hi + c.pH) * c.Wo + wi + c.pW);
            ph[u] = FAST ? hi + c.pH : hi;
            pw[u] = FAST ? wi + c.pW : wi;
          } else {
            nb[u] = 0; ph[u] = 0; pw[u] = 0;
          }
          if (++wi == c.W) { wi = 0; if (++hi == c.H) { hi = 0; ++b; } }
        }
      }
    } else {
      const int khw = c.kH * c.kW;
      for (int e = 0; e < QB; ++e) {
        int rr, kk;
        stage_coords_rt(e, rr, kk);
        const int n = p.n0 + rr;
        if (n < c.N) {
          wnvalid |= 1 << e;
          const int cl = fdiv(n, c.dKHW), r = n - cl * khw;
          const int kh = fdiv(r, c.dKW), kw = r - kh * c.kW;
          wdh[e] = kh - c.pH;
          wdw[e] = kw - c.pW;
          wnoff[e] = (uint32_t)(((p.z * c.CinPG + cl) * c.H) * c.W) + (uint32_t)(wdh[e] * c.W + wdw[e]);
        } else {
          wdh[e] = 0; wdw[e] = 0; wnoff[e] = 0;
        }
      }
    }
  }

  // Runtime-index version of stage_coords for the KFAST B operand.
  CG_HD void stage_coords_rt(int e, int& rr, int& kk) const {
    const int idx = tid + e * kCT;
    rr = idx / (kCBK / 4);
    kk = (idx % (kCBK / 4)) * 4;
  }

  // A operand (always k-contiguous): 4 consecutive k of row m.
  CG_HD f32x4 load_a(const ConvGemmArgs& c, int m, int k0) const {
    f32x4 v;
    const int kend = bp.kend;
    const bool mok = m < c.M;
    const int mm = mok ? m : 0;
    if ((F & F_TAP) && MODE != CV_WGRAD) {
      // k = tap * cpg + ch; the 4 k share the tap (cpg % 4 == 0, k0 % 4 == 0) and lie below
      // kend (K = taps * cpg, a multiple of kCBK). Consecutive channels are a fixed stride
      // apart in the weight.
      const int khw = c.kH * c.kW;
      const int cpg = MODE == CV_FWD ? c.CinPG : c.CoutPG;
      const int tap = fdiv(k0, c.dCpg), ch = k0 - tap * cpg;
      const uint32_t o = MODE == CV_FWD ? (uint32_t)(((bp.z * c.CoutPG + mm) * c.CinPG + ch) * khw + tap)
                                        : (uint32_t)(((bp.z * c.CoutPG + ch) * c.CinPG + mm) * khw + tap);
      const uint32_t step = MODE == CV_FWD ? (uint32_t)khw : (uint32_t)(c.CinPG * khw);
      for (int u = 0; u < 4; ++u) v[u] = ldb(sw, mok ? (o + u * step) << 2 : kMasked);
      (void)kend;
      return v;
    }
    if (MODE == CV_FWD) {
      const uint32_t row = (uint32_t)((bp.z * c.CoutPG + mm) * c.K);
      // avec: K % 4 == 0 and k0 % 4 == 0, so k0 < kend covers all 4
      if (F & F_AVEC) return ldb4(sw, boff(mok && k0 < kend, row + (uint32_t)k0));
      for (int u = 0; u < 4; ++u) v[u] = ldb(sw, boff(mok && k0 + u < kend, row + (uint32_t)(k0 + u)));
    } else if (MODE == CV_DGRAD) {
      const int khw = c.kH * c.kW;
      int col = fdiv(k0, c.dKHW), r = k0 - col * khw;
      for (int u = 0; u < 4; ++u) {
        const bool ok = mok && k0 + u < kend;
        v[u] = ldb(sw, boff(ok, (uint32_t)(((bp.z * c.CoutPG + (ok ? col : 0)) * c.CinPG + mm) * khw + r)));
        if (++r == khw) { r = 0; ++col; }
      }
    } else {   // CV_WGRAD: dy[b, co, p] for k = (b, p)
      const int hw = c.Ho * c.Wo;
      const bool kok = k0 < kend;
      int b = kok ? fdiv(k0, c.dHoWo) : 0, p = kok ? k0 - b * hw : 0;
      // avec: hw % 4 == 0 and k0 % 4 == 0, so the 4 k lie in one image, 16-byte aligned
      if (F & F_AVEC) return ldb4(sdy, boff(mok && kok, (uint32_t)((b * c.Cout + bp.z * c.CoutPG + mm) * hw + p)));
      for (int u = 0; u < 4; ++u) {
        const bool ok = mok && k0 + u < kend;
        v[u] = ldb(sdy, boff(ok, (uint32_t)(((ok ? b : 0) * c.Cout + bp.z * c.CoutPG + mm) * hw + (ok ? p : 0))));
        if (++p == hw) { p = 0; ++b; }
      }
    }
    return v;
  }

  // Row-contiguous B (conv2d, input gradient): the thread's 4 positions at one k. `tab`
  // holds (offset, shifts) of every k when K <= kTab (else null: computed here).
  CG_HD f32x4 load_b_rows(const ConvGemmArgs& c, int k, const uint32_t* tab) const {
    f32x4 v;
    const bool kok = k < bp.kend;
    const int kq = kok ? k : 0;
    if (MODE == CV_FWD || FAST) {
      uint32_t koff, sh;
      if (F & F_TAB) { koff = tab[2 * kq]; sh = tab[2 * kq + 1]; }
      else k_term(c, MODE, kq, koff, sh);
      const int a = shift_lo(sh), b = shift_hi(sh);
      const Src& src = MODE == CV_FWD ? sx : sdy;
      for (int u = 0; u < 4; ++u) {
        bool ok = kok && ((nvalid >> u) & 1);
        if (MODE == CV_FWD) {
          if (F & F_PAD) ok = ok && inside(ph[u] + a, c.H) && inside(pw[u] + b, c.W);
        } else {
          ok = ok && inside(ph[u] - a, c.Ho) && inside(pw[u] - b, c.Wo);
        }
        v[u] = ldb(src, boff(ok, nb[u] + koff));
      }
    } else {             // input gradient, any stride: ph / pw hold (hi, wi)
      const int khw = c.kH * c.kW;
      const int kc = fdiv(kq, c.dKHW), r = kq - kc * khw;
      const int kh = fdiv(r, c.dKW), kw = r - kh * c.kW;
      for (int u = 0; u < 4; ++u) {
        const int nh = ph[u] + c.pH - kh, nw = pw[u] + c.pW - kw;
        bool ok = kok && ((nvalid >> u) & 1) && nh >= 0 && nw >= 0;
        const int ho = fdiv(ok ? nh : 0, c.dSH), wo = fdiv(ok ? nw : 0, c.dSW);
        ok = ok && ho * c.sH == nh && wo * c.sW == nw && ho < c.Ho && wo < c.Wo;
        // nb[u] - (hi + pH) * Wo - (wi + pW) is the (b, g) plane base
        const uint32_t plane = nb[u] - (uint32_t)((ph[u] + c.pH) * c.Wo + pw[u] + c.pW);
        v[u] = ldb(sdy, boff(ok, plane + (uint32_t)(kc * c.Ho * c.Wo + ho * c.Wo + wo)));
      }
    }
    return v;
  }

  // k-contiguous B (weight gradient): group e's column at 4 consecutive k = (b, ho, wo).
  // kb/khs/kws: the per-stage k terms (position term, spatial coordinates) of the 4 k.
  CG_HD f32x4 load_b_cols(const ConvGemmArgs& c, int e, const uint32_t* kb, const int* khs, const int* kws,
                          int kmask) const {
    f32x4 v;
    const bool nok = (wnvalid >> e) & 1;
    for (int u = 0; u < 4; ++u) {
      bool ok = nok && ((kmask >> u) & 1);
      if (F & F_PAD) ok = ok && inside(khs[u] + wdh[e], c.H) && inside(kws[u] + wdw[e], c.W);
      v[u] = ldb(sx, boff(ok, kb[u] + wnoff[e]));
    }
    return v;
  }

  // One stage: fill qa[QA] / qb[QB] with the elements this thread stages for k0.
  CG_HD void load(const ConvGemmArgs& c, int k0, f32x4* qa, f32x4* qb, const uint32_t* tab) const {
    for (int e = 0; e < QA; ++e) {
      const int idx = tid + e * kCT;
      const int rr = idx / (kCBK / 4), kk = (idx % (kCBK / 4)) * 4;
      qa[e] = load_a(c, bp.m0 + rr, k0 + kk);
    }
    if (!BKF && (F & F_TAP)) {
      // The stage's 32 k are one tap (cpg % kCBK == 0, k0 % kCBK == 0, K = taps * cpg, so
      // every k < kend): in-image tests and offset bases per position once, then per k the
      // channel's plane offset. Masked positions keep the out-of-range base kMasked, which
      // the added plane offset (below 2^31 bytes) leaves out of range.
      const int cpg = MODE == CV_FWD ? c.CinPG : c.CoutPG;
      const int tap = fdiv(k0, c.dCpg);
      const int kh = fdiv(tap, c.dKW), kw = tap - kh * c.kW;
      const int a = MODE == CV_FWD ? kh - c.pH : kh, b = MODE == CV_FWD ? kw - c.pW : kw;
      const uint32_t toff = MODE == CV_FWD ? (uint32_t)(a * c.W + b) : (uint32_t)0 - (uint32_t)(kh * c.Wo + kw);
      const uint32_t plane = MODE == CV_FWD ? (uint32_t)(c.H * c.W) : (uint32_t)(c.Ho * c.Wo);
      const Src& src = MODE == CV_FWD ? sx : sdy;
      uint32_t base[4];
      for (int u = 0; u < 4; ++u) {
        bool ok = (nvalid >> u) & 1;
        if (MODE == CV_FWD) {
          if (F & F_PAD) ok = ok && inside(ph[u] + a, c.H) && inside(pw[u] + b, c.W);
        } else {
          ok = ok && inside(ph[u] - a, c.Ho) && inside(pw[u] - b, c.Wo);
        }
        base[u] = ok ? (nb[u] + toff) << 2 : kMasked;
      }
      const int ch0 = k0 - tap * cpg;
      for (int e = 0; e < QB; ++e) {
        const int kk = (tid + e * kCT) / (BN / 4);
        const uint32_t delta = ((uint32_t)(ch0 + kk) * plane) << 2;
        for (int u = 0; u < 4; ++u) qb[e][u] = ldb(src, base[u] + delta);
      }
    } else if (!BKF) {
      for (int e = 0; e < QB; ++e) {
        const int idx = tid + e * kCT;
        const int kk = idx / (BN / 4);
        qb[e] = load_b_rows(c, k0 + kk, tab);
      }
    } else {
      // The thread's 4 k are the same for every group (kk depends on tid only).
      const int kk = (tid % (kCBK / 4)) * 4;
      uint32_t kb[4];
      int khs[4], kws[4], kmask = 0;
      const int hw = c.Ho * c.Wo;
      const int ks = k0 + kk;
      int b = 0, p = 0;
      if (ks < bp.kend) { b = fdiv(ks, c.dHoWo); p = ks - b * hw; }
      int ho = fdiv(p, c.dWo), wo = p - ho * c.Wo;
      for (int u = 0; u < 4; ++u) {
        if (ks + u < bp.kend) kmask |= 1 << u;
        kb[u] = (uint32_t)((b * c.Cin * c.H + ho * c.sH) * c.W + wo * c.sW);
        khs[u] = ho * c.sH;
        kws[u] = wo * c.sW;
        if (++wo == c.Wo) { wo = 0; if (++ho == c.Ho) { ho = 0; ++b; } }
      }
      for (int e = 0; e < QB; ++e) qb[e] = load_b_cols(c, e, kb, khs, kws, kmask);
    }
  }

  // Output offset of GEMM element (0, gn) and the stride between rows gm (for split-K
  // weight gradients, the offset inside the split's partial tile array).
  CG_HD int64_t out_col(const ConvGemmArgs& c, int gn) const {
    if (MODE == CV_FWD) {
      const int hw = c.Ho * c.Wo;
      const int b = fdiv(gn, c.dHoWo), q = gn - b * hw;
      return ((int64_t)b * c.Cout + bp.z * c.CoutPG) * hw + q;
    }
    if (MODE == CV_DGRAD) {
      const int hw = c.H * c.W;
      const int b = fdiv(gn, c.dHW), q = gn - b * hw;
      return ((int64_t)b * c.Cin + bp.z * c.CinPG) * hw + q;
    }
    if (c.splits > 1) return ((int64_t)bp.split * c.G + bp.z) * c.M * c.N + gn;
    return (int64_t)bp.z * c.M * c.N + gn;
  }
  CG_HD int64_t out_rs(const ConvGemmArgs& c) const {
    return MODE == CV_FWD ? (int64_t)c.Ho * c.Wo : MODE == CV_DGRAD ? (int64_t)c.H * c.W : (int64_t)c.N;
  }
};

struct ConvPlan { int mode, bm, bn, splits, k_per_split, tiles_m, tiles_n; int64_t blocks; };

inline ConvPlan conv_plan(int mode, const ConvDesc& d) {
  ConvPlan p{};
  p.mode = mode;
  const int64_t CoutPG = d.Cout / d.G, khw = d.kH * d.kW;
  const int64_t M = mode == CV_DGRAD ? d.CinPG : CoutPG;
  const int64_t N = mode == CV_FWD ? d.B * d.Ho * d.Wo : mode == CV_DGRAD ? d.B * d.H * d.W : d.CinPG * khw;
  const int64_t K = mode == CV_FWD ? d.CinPG * khw : mode == CV_DGRAD ? CoutPG * khw : d.B * d.Ho * d.Wo;
  const int64_t Z = d.G;
  // Tiles measured at the CNN config's shapes: 64 x 64 where M > 32 (more blocks in
  // flight than 64 x 128 at the same per-element cost), 32 x 128 for 32-row outputs.
  p.bm = M <= 32 ? 32 : 64;
  p.bn = p.bm == 32 ? 128 : 64;
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
  const int khw = a.kH * a.kW;
  if (p.mode == CV_FWD) { a.M = a.CoutPG; a.N = a.B * a.Ho * a.Wo; a.K = a.CinPG * khw; }
  else if (p.mode == CV_DGRAD) { a.M = a.CinPG; a.N = a.B * a.H * a.W; a.K = a.CoutPG * khw; }
  else { a.M = a.CoutPG; a.N = a.CinPG * khw; a.K = a.B * a.Ho * a.Wo; }
  a.tiles_m = p.tiles_m; a.tiles_n = p.tiles_n; a.splits = p.splits; a.k_per_split = p.k_per_split;
  // A tap outside the image exists iff padding is used or the last window overhangs.
  // (pad, avec and whether the k table applies select the loader variant, see F_*.)
  a.pad = (a.pH > 0 || a.pW > 0 || (a.Ho - 1) * a.sH + a.kH > a.H || (a.Wo - 1) * a.sW + a.kW > a.W) ? 1 : 0;
  a.avec = p.mode == CV_FWD ? (a.K % 4 == 0) : p.mode == CV_WGRAD ? ((a.Ho * a.Wo) % 4 == 0) : 0;   // and aligned bases (set with the pointers)
  a.dKHW = make_fastdiv((uint32_t)khw);
  a.dKW = make_fastdiv((uint32_t)a.kW);
  a.dWo = make_fastdiv((uint32_t)a.Wo);
  a.dHoWo = make_fastdiv((uint32_t)(a.Ho * a.Wo));
  a.dW = make_fastdiv((uint32_t)a.W);
  a.dHW = make_fastdiv((uint32_t)(a.H * a.W));
  a.dSH = make_fastdiv((uint32_t)a.sH);
  a.dSW = make_fastdiv((uint32_t)a.sW);
  a.dCpg = make_fastdiv((uint32_t)(p.mode == CV_FWD ? a.CinPG : a.CoutPG));
  return a;
}

// Loader flags of a launch (avec must already account for the operand's alignment).
inline int conv_flags(const ConvGemmArgs& a, int mode) {
  // Tap-major order for the stride-1 input gradient only: measured on the CNN config it
  // cuts the input gradient's index arithmetic (72.7 -> 63.8 us) but slows conv2d, whose
  // k-contiguous weight rows then lose their vector loads and whose stages read 32
  // channel planes instead of a few neighbouring rows (43.7 -> 68.9 us).
  const bool tap = mode == CV_DGRAD && a.sH == 1 && a.sW == 1 && a.CoutPG % kCBK == 0;
  if (tap) return F_TAP;
  int f = 0;
  if (a.avec && mode != CV_DGRAD) f |= F_AVEC;
  if (a.pad && mode != CV_DGRAD) f |= F_PAD;
  if ((mode == CV_FWD || mode == CV_DGRAD) && a.K <= kTab) f |= F_TAB;
  return f;
}

// Every tensor, offset and launch indexable in 32 bits, and a geometry the maps assume.
inline bool conv_ok(const ConvDesc& d) {
  const int64_t lim = int64_t(1) << 29;
  if (d.B <= 0 || d.G <= 0 || d.Cout % d.G != 0 || d.sH <= 0 || d.sW <= 0 || d.Ho <= 0 || d.Wo <= 0 || d.kH <= 0 ||
      d.kW <= 0 || d.pH < 0 || d.pW < 0 || d.H <= 0 || d.W <= 0)
    return false;
  // the position terms of the input gradient reach (b, g*CoutPG, Ho + pH, Wo + pW)
  const int64_t big = std::max({d.B * d.Cin * d.H * d.W, d.B * d.Cout * d.Ho * d.Wo, d.Cout * d.CinPG * d.kH * d.kW,
                                d.B * d.Cout * (d.Ho + d.H + d.pH + 1) * (d.Wo + d.W + d.pW + 1),
                                (d.H + d.pH + d.kH) * (d.W + d.pW + d.kW)});
  if (big >= lim) return false;
  for (int mode : {CV_FWD, CV_DGRAD, CV_WGRAD})
    if (conv_plan(mode, d).blocks >= lim) return false;
  return true;
}

#undef CG_HD

}  // namespace cg
}  // namespace tgk
