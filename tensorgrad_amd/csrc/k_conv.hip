// Direct NCHW convolution and max-pool kernels for gfx950.
//
// conv2d and its input gradient run one thread per output element and accumulate in
// f64 over (input channel, kh, kw) in the reference evaluator's order
// (test/_eval.ts:619-684), so they reproduce the CPU evaluation exactly; the f64 FMA
// gives the same result as the evaluator's separate multiply-add because a product of
// two f32 values is exact in f64. The weight gradient reduces B*Ho*Wo terms per weight
// with one 256-thread block per weight element, f64 partial sums combined in a fixed
// tree (deterministic). Pooling keeps the evaluator's -3.4e38 initial value and strict
// `>` scan order (ties resolve to the first element scanned, _eval.ts:716-779).
#include "kernels.h"

namespace tgk {
namespace {

inline int grid_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  return (int)(b > 8192 ? 8192 : (b < 1 ? 1 : b));
}

__global__ void k_conv2d(const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ y, ConvDesc c) {
  const int64_t total = c.B * c.Cout * c.Ho * c.Wo;
  const int64_t coutPG = c.Cout / c.G;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t wo = i % c.Wo, t = i / c.Wo;
    int64_t ho = t % c.Ho; t /= c.Ho;
    int64_t co = t % c.Cout, b = t / c.Cout;
    int64_t g = co / coutPG;
    double s = 0.0;
    for (int64_t cl = 0; cl < c.CinPG; ++cl) {
      const int64_t ci = g * c.CinPG + cl;
      for (int64_t kh = 0; kh < c.kH; ++kh) {
        const int64_t hi = ho * c.sH + kh - c.pH;
        if (hi < 0 || hi >= c.H) continue;
        for (int64_t kw = 0; kw < c.kW; ++kw) {
          const int64_t wi = wo * c.sW + kw - c.pW;
          if (wi < 0 || wi >= c.W) continue;
          s = fma((double)x[((b * c.Cin + ci) * c.H + hi) * c.W + wi],
                  (double)w[((co * c.CinPG + cl) * c.kH + kh) * c.kW + kw], s);
        }
      }
    }
    y[i] = (float)s;
  }
}

__global__ void k_conv2d_dx(const float* __restrict__ w, const float* __restrict__ dy, float* __restrict__ dx,
                            ConvDesc c) {
  const int64_t total = c.B * c.Cin * c.H * c.W;
  const int64_t coutPG = c.Cout / c.G;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t wi = i % c.W, t = i / c.W;
    int64_t hi = t % c.H; t /= c.H;
    int64_t ci = t % c.Cin, b = t / c.Cin;
    int64_t g = ci / c.CinPG, cl = ci - g * c.CinPG;
    double s = 0.0;
    for (int64_t col = 0; col < coutPG; ++col) {
      const int64_t co = g * coutPG + col;
      for (int64_t kh = 0; kh < c.kH; ++kh) {
        const int64_t nh = hi + c.pH - kh;
        if (nh < 0 || nh % c.sH != 0) continue;
        const int64_t ho = nh / c.sH;
        if (ho >= c.Ho) continue;
        for (int64_t kw = 0; kw < c.kW; ++kw) {
          const int64_t nw = wi + c.pW - kw;
          if (nw < 0 || nw % c.sW != 0) continue;
          const int64_t wo = nw / c.sW;
          if (wo >= c.Wo) continue;
          s = fma((double)w[((co * c.CinPG + cl) * c.kH + kh) * c.kW + kw],
                  (double)dy[((b * c.Cout + co) * c.Ho + ho) * c.Wo + wo], s);
        }
      }
    }
    dx[i] = (float)s;
  }
}

// One block per weight element; threads stride over (b, ho, wo).
__global__ __launch_bounds__(256) void k_conv2d_dw(const float* __restrict__ x, const float* __restrict__ dy,
                                                   float* __restrict__ dw, ConvDesc c) {
  __shared__ double red[256];
  const int64_t nW = c.Cout * c.CinPG * c.kH * c.kW;
  const int64_t coutPG = c.Cout / c.G;
  const int64_t span = c.B * c.Ho * c.Wo;
  for (int64_t e = blockIdx.x; e < nW; e += gridDim.x) {
    int64_t kw = e % c.kW, t = e / c.kW;
    int64_t kh = t % c.kH; t /= c.kH;
    int64_t cl = t % c.CinPG, co = t / c.CinPG;
    int64_t ci = (co / coutPG) * c.CinPG + cl;
    double s = 0.0;
    for (int64_t q = threadIdx.x; q < span; q += blockDim.x) {
      int64_t wo = q % c.Wo, u = q / c.Wo;
      int64_t ho = u % c.Ho, b = u / c.Ho;
      int64_t hi = ho * c.sH + kh - c.pH, wi = wo * c.sW + kw - c.pW;
      if (hi < 0 || hi >= c.H || wi < 0 || wi >= c.W) continue;
      s = fma((double)x[((b * c.Cin + ci) * c.H + hi) * c.W + wi], (double)dy[((b * c.Cout + co) * c.Ho + ho) * c.Wo + wo], s);
    }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
      if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
      __syncthreads();
    }
    if (threadIdx.x == 0) dw[e] = (float)red[0];
    __syncthreads();
  }
}

__global__ void k_max_pool(const float* __restrict__ x, float* __restrict__ y, PoolDesc p) {
  const int64_t total = p.B * p.C * p.Ho * p.Wo;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t wo = i % p.Wo, t = i / p.Wo;
    int64_t ho = t % p.Ho, bc = t / p.Ho;
    const float* plane = x + bc * p.H * p.W;
    float m = -3.4e38f;
    for (int64_t kh = 0; kh < p.kH; ++kh) {
      int64_t hi = ho * p.sH + kh - p.pH;
      if (hi < 0 || hi >= p.H) continue;
      for (int64_t kw = 0; kw < p.kW; ++kw) {
        int64_t wi = wo * p.sW + kw - p.pW;
        if (wi < 0 || wi >= p.W) continue;
        float v = plane[hi * p.W + wi];
        if (v > m) m = v;
      }
    }
    y[i] = m;
  }
}

// Gather form of the pool adjoint: each input element collects dy from every window
// whose (recomputed) argmax is this element.
__global__ void k_max_pool_grad(const float* __restrict__ x, const float* __restrict__ dy, float* __restrict__ dx,
                                PoolDesc p, bool relu) {
  const int64_t total = p.B * p.C * p.H * p.W;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t wi = i % p.W, t = i / p.W;
    int64_t hi = t % p.H, bc = t / p.H;
    const float* plane = x + bc * p.H * p.W;
    double s = 0.0;
    for (int64_t kh = 0; kh < p.kH; ++kh) {
      int64_t nh = hi + p.pH - kh;
      if (nh < 0 || nh % p.sH != 0) continue;
      int64_t ho = nh / p.sH;
      if (ho >= p.Ho) continue;
      for (int64_t kw = 0; kw < p.kW; ++kw) {
        int64_t nw = wi + p.pW - kw;
        if (nw < 0 || nw % p.sW != 0) continue;
        int64_t wo = nw / p.sW;
        if (wo >= p.Wo) continue;
        float m = -3.4e38f;
        int64_t ah = -1, aw = -1;
        for (int64_t kkh = 0; kkh < p.kH; ++kkh) {
          int64_t hh = ho * p.sH + kkh - p.pH;
          if (hh < 0 || hh >= p.H) continue;
          for (int64_t kkw = 0; kkw < p.kW; ++kkw) {
            int64_t ww = wo * p.sW + kkw - p.pW;
            if (ww < 0 || ww >= p.W) continue;
            float v = plane[hh * p.W + ww];
            if (v > m) { m = v; ah = hh; aw = ww; }
          }
        }
        if (ah == hi && aw == wi) s += (double)dy[(bc * p.Ho + ho) * p.Wo + wo];
      }
    }
    dx[i] = relu && !(plane[hi * p.W + wi] > 0.0f) ? 0.0f : (float)s;
  }
}

// Pooling with 32-bit indexing (every tensor below 2^31 elements): one thread per window,
// the same scan as k_max_pool (row-major over the window, -3.4e38 start, strict `>`).
struct Pool32 {
  int H, W, Ho, Wo, kH, kW, sH, sW, pH, pW;
  int64_t nwin;
  FastDiv dWo, dHoWo;
};

__device__ __forceinline__ void window_of(const Pool32& p, int i, int& bc, int& ho, int& wo) {
  bc = (int)fastdiv((uint32_t)i, p.dHoWo);
  const int q = i - bc * p.Ho * p.Wo;
  ho = (int)fastdiv((uint32_t)q, p.dWo);
  wo = q - ho * p.Wo;
}

__global__ void k_max_pool32(const float* __restrict__ x, float* __restrict__ y, Pool32 p) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < p.nwin; i += gridDim.x * blockDim.x) {
    int bc, ho, wo;
    window_of(p, i, bc, ho, wo);
    const float* plane = x + (int64_t)bc * p.H * p.W;
    float m = -3.4e38f;
    for (int kh = 0; kh < p.kH; ++kh) {
      const int hi = ho * p.sH + kh - p.pH;
      if (hi < 0 || hi >= p.H) continue;
      for (int kw = 0; kw < p.kW; ++kw) {
        const int wi = wo * p.sW + kw - p.pW;
        if (wi < 0 || wi >= p.W) continue;
        const float v = plane[hi * p.W + wi];
        if (v > m) m = v;
      }
    }
    y[i] = m;
  }
}

// Adjoint when the windows tile the input exactly (stride = window, no padding, H = Ho*sH,
// W = Wo*sW): every input element lies in exactly one window, so each window writes its
// own elements: dy at the recomputed argmax (the first maximum in scan order), zero
// elsewhere. Equal to the gather form bit for bit (one term per element). With `relu` the
// ReLU gradient of the pooled input follows: only the argmax element can be non-zero, and
// its mask is the window's maximum > 0 (+0 where it is not, NaN included).
__global__ void k_max_pool_grad_tiled(const float* __restrict__ x, const float* __restrict__ dy,
                                      float* __restrict__ dx, Pool32 p, bool relu) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < p.nwin; i += gridDim.x * blockDim.x) {
    int bc, ho, wo;
    window_of(p, i, bc, ho, wo);
    const int64_t base = (int64_t)bc * p.H * p.W;
    float m = -3.4e38f;
    int arg = -1;
    for (int kh = 0; kh < p.kH; ++kh)
      for (int kw = 0; kw < p.kW; ++kw) {
        const int off = (ho * p.sH + kh) * p.W + wo * p.sW + kw;
        const float v = x[base + off];
        if (v > m) { m = v; arg = off; }
      }
    const float g = relu && !(m > 0.0f) ? 0.0f : dy[i];
    for (int kh = 0; kh < p.kH; ++kh)
      for (int kw = 0; kw < p.kW; ++kw) {
        const int off = (ho * p.sH + kh) * p.W + wo * p.sW + kw;
        dx[base + off] = off == arg ? g : 0.0f;
      }
  }
}

// 2 x 2 windows with stride 2 tiling the input (H = 2 Ho, W = 2 Wo, no padding; the
// CNN's pools): the same scan order and comparisons as above, a window's two input rows as
// one 8-byte load each (both loads in flight before the comparisons).
__device__ __forceinline__ const float2* pool22_rows(const float* x, const Pool32& p, int bc, int ho, int wo,
                                                    int64_t& base) {
  base = (int64_t)bc * p.H * p.W + (int64_t)(2 * ho) * p.W + 2 * wo;
  return reinterpret_cast<const float2*>(x + base);
}

__global__ void k_max_pool22(const float* __restrict__ x, float* __restrict__ y, Pool32 p) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < p.nwin; i += gridDim.x * blockDim.x) {
    int bc, ho, wo;
    window_of(p, i, bc, ho, wo);
    int64_t base;
    const float2* r = pool22_rows(x, p, bc, ho, wo, base);
    const float2 a = r[0], b = *reinterpret_cast<const float2*>(x + base + p.W);
    float m = -3.4e38f;
    if (a.x > m) m = a.x;
    if (a.y > m) m = a.y;
    if (b.x > m) m = b.x;
    if (b.y > m) m = b.y;
    y[i] = m;
  }
}

__global__ void k_max_pool22_grad(const float* __restrict__ x, const float* __restrict__ dy,
                                  float* __restrict__ dx, Pool32 p, bool relu) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < p.nwin; i += gridDim.x * blockDim.x) {
    int bc, ho, wo;
    window_of(p, i, bc, ho, wo);
    int64_t base;
    const float2* r = pool22_rows(x, p, bc, ho, wo, base);
    const float2 a = r[0], b = *reinterpret_cast<const float2*>(x + base + p.W);
    const float g = dy[i];
    float m = -3.4e38f;
    int arg = -1;
    if (a.x > m) { m = a.x; arg = 0; }
    if (a.y > m) { m = a.y; arg = 1; }
    if (b.x > m) { m = b.x; arg = 2; }
    if (b.y > m) { m = b.y; arg = 3; }
    if (relu && !(m > 0.0f)) arg = -1;   // the ReLU gradient of the pooled input (see above)
    *reinterpret_cast<float2*>(dx + base) = make_float2(arg == 0 ? g : 0.0f, arg == 1 ? g : 0.0f);
    *reinterpret_cast<float2*>(dx + base + p.W) = make_float2(arg == 2 ? g : 0.0f, arg == 3 ? g : 0.0f);
  }
}

bool pool22(const PoolDesc& d, const void* a, const void* b) {
  return d.kH == 2 && d.kW == 2 && d.sH == 2 && d.sW == 2 && d.pH == 0 && d.pW == 0 && d.H == 2 * d.Ho &&
         d.W == 2 * d.Wo && ((uintptr_t)a & 7) == 0 && ((uintptr_t)b & 7) == 0;
}

Pool32 pool32(const PoolDesc& d) {
  Pool32 p{};
  p.H = (int)d.H; p.W = (int)d.W; p.Ho = (int)d.Ho; p.Wo = (int)d.Wo; p.kH = (int)d.kH; p.kW = (int)d.kW;
  p.sH = (int)d.sH; p.sW = (int)d.sW; p.pH = (int)d.pH; p.pW = (int)d.pW;
  p.nwin = d.B * d.C * d.Ho * d.Wo;
  p.dWo = make_fastdiv((uint32_t)d.Wo);
  p.dHoWo = make_fastdiv((uint32_t)(d.Ho * d.Wo));
  return p;
}

bool pool_small(const PoolDesc& d) {
  return d.B * d.C * d.H * d.W < (int64_t(1) << 31) && d.B * d.C * d.Ho * d.Wo < (int64_t(1) << 31) && d.Ho > 0 &&
         d.Wo > 0;
}

}  // namespace

void conv2d(const float* x, const float* w, float* y, const ConvDesc& c, hipStream_t st) {
  int64_t n = c.B * c.Cout * c.Ho * c.Wo;
  if (n <= 0) return;
  klaunch(k_conv2d, grid_for(n), 256, 0, st, x, w, y, c);
}

void conv2d_input_grad(const float* w, const float* dy, float* dx, const ConvDesc& c, hipStream_t st) {
  int64_t n = c.B * c.Cin * c.H * c.W;
  if (n <= 0) return;
  klaunch(k_conv2d_dx, grid_for(n), 256, 0, st, w, dy, dx, c);
}

int64_t conv2d_weight_grad_workspace(const ConvDesc&) { return 0; }

void conv2d_weight_grad(const float* x, const float* dy, float* dw, const ConvDesc& c, double*, hipStream_t st) {
  int64_t nW = c.Cout * c.CinPG * c.kH * c.kW;
  if (nW <= 0) return;
  int64_t blocks = nW < 65536 ? nW : 65536;
  klaunch(k_conv2d_dw, (int)blocks, 256, 0, st, x, dy, dw, c);
}

void max_pool(const float* x, float* y, const PoolDesc& p, hipStream_t st) {
  int64_t n = p.B * p.C * p.Ho * p.Wo;
  if (n <= 0) return;
  if (pool_small(p)) {
    if (pool22(p, x, x)) klaunch(k_max_pool22, grid_for(n), 256, 0, st, x, y, pool32(p));
    else klaunch(k_max_pool32, grid_for(n), 256, 0, st, x, y, pool32(p));
    return;
  }
  klaunch(k_max_pool, grid_for(n), 256, 0, st, x, y, p);
}

void max_pool_grad(const float* x, const float* dy, float* dx, const PoolDesc& p, hipStream_t st, bool relu) {
  int64_t n = p.B * p.C * p.H * p.W;
  if (n <= 0) return;
  const bool tiled = p.sH == p.kH && p.sW == p.kW && p.pH == 0 && p.pW == 0 && p.H == p.Ho * p.sH &&
                     p.W == p.Wo * p.sW;
  if (tiled && pool_small(p)) {
    if (pool22(p, x, dx))
      klaunch(k_max_pool22_grad, grid_for(p.B * p.C * p.Ho * p.Wo), 256, 0, st, x, dy, dx, pool32(p), relu);
    else klaunch(k_max_pool_grad_tiled, grid_for(p.B * p.C * p.Ho * p.Wo), 256, 0, st, x, dy, dx, pool32(p), relu);
    return;
  }
  klaunch(k_max_pool_grad, grid_for(n), 256, 0, st, x, dy, dx, p, relu);
}

}  // namespace tgk
