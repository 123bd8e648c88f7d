// Host-side launch wrappers for the gfx950 kernels. Each wrapper enqueues one kernel on
// `st`; shapes arrive as plain integers (no torch types). All element storage is 4-byte:
// f32, or i32 for the `i32` and `bool` IR dtypes.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <cstdint>
#include <vector>

#include "fused_dev.h"
#include "gemm_dev.h"

namespace tgk {

constexpr int kMaxRank = 8;

// Kernel timing for measurement (tg_profile_kernels): while a timer is installed on the
// calling thread, each launch records the kernel's own start and end timestamps (those of
// its dispatch packet, the quantity a profiler's kernel trace reports) into a pair of
// events from the timer's pool; otherwise it is a plain launch.
struct LaunchTimer {
  std::vector<hipEvent_t> ev;   // pairs: ev[2i] start, ev[2i + 1] end
  size_t used = 0;              // pairs handed out
  size_t missed = 0;            // launches left untimed (pool exhausted)
  bool take(hipEvent_t& a, hipEvent_t& b) {
    if (2 * used + 1 >= ev.size()) { ++missed; return false; }
    a = ev[2 * used];
    b = ev[2 * used + 1];
    ++used;
    return true;
  }
};
LaunchTimer*& launch_timer();   // the calling thread's installed timer (null: none)

template <typename... Args, typename F = void (*)(Args...)>
inline void klaunch(F kernel, const dim3& grid, const dim3& block, uint32_t lds, hipStream_t st, Args... args) {
  hipEvent_t a = nullptr, b = nullptr;
  LaunchTimer* t = launch_timer();
  if (t && t->take(a, b)) {
    hipExtLaunchKernelGGL(kernel, grid, block, lds, st, a, b, 0, args...);
    return;
  }
  hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
}

// Division by a runtime constant d >= 1 for 0 <= x < 2^31 without a divide instruction:
// q = (umulhi(x, m) + x) >> s with s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1
// (Granlund & Montgomery, "Division by invariant integers using multiplication", 1994).
// umulhi(x, m) <= x, so the sum stays below 2^32.
struct FastDiv {
  uint32_t d, m, s;
};
inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{d, 0, 0};
  while ((1ull << f.s) < d) ++f.s;
  f.m = (uint32_t)((((1ull << 32) * ((1ull << f.s) - d)) / d) + 1);
  return f;
}
__device__ __forceinline__ uint32_t fastdiv(uint32_t x, const FastDiv& f) {
  return (__umulhi(x, f.m) + x) >> f.s;
}

// An N-d iteration space with per-operand element strides (0 = broadcast axis).
struct Strided {
  int rank;
  int64_t dims[kMaxRank];
  int64_t s0[kMaxRank];   // operand 0 strides
  int64_t s1[kMaxRank];   // operand 1 strides
  int64_t s2[kMaxRank];   // operand 2 strides
};

// ---- element-wise (k_elementwise.hip) -----------------------------------------------
enum BinOp { B_ADD, B_SUB, B_MUL, B_DIV, B_MIN, B_MAX, B_LESS, B_GREATER };
enum UnOp { U_SQRT, U_RSQRT, U_LOG, U_EXP, U_RELU, U_NEG, U_ABS, U_TANH, U_SIGMOID, U_ERF, U_SIN, U_COS };

// out[i] = a[.] op b[.] over `sp` (operand 0 = a, 1 = b); out is contiguous.
void binary(int op, const void* a, int a_dt, const void* b, int b_dt, void* out, int out_dt, const Strided& sp,
            int64_t n, hipStream_t st);
// out[i] = f32(a[i] * s) or f32(a[i] + s), f64 arithmetic.
void scalar_op(bool mul, const void* a, int a_dt, double s, float* out, int64_t n, hipStream_t st);
void unary(int op, const float* a, float* out, int64_t n, hipStream_t st);
void relu_grad(const float* x, const float* dy, float* out, int64_t n, hipStream_t st);
// out = cond ? a : b with broadcast strides (operand 0 = cond, 1 = a, 2 = b).
void where(const int32_t* cond, const void* a, const void* b, int dt, void* out, const Strided& sp, int64_t n,
           hipStream_t st);
void where_causal(const float* a, float* out, int64_t outer, int64_t D, double fill, hipStream_t st);
// dst[strided] = src[strided]: permute / broadcast_to / slice / concat / scatter.
// Operand 0 = dst strides, operand 1 = src strides; both 4-byte elements.
void strided_copy(void* dst, const void* src, const Strided& sp, int64_t n, hipStream_t st);
// Concatenation along the last axis of n <= kConcatMax contiguous [rows, w_i] inputs into a
// contiguous [rows, W] output (W = sum w_i), one launch writing the output in order.
constexpr int kConcatMax = 8;
struct ConcatLast {
  int n;
  const uint32_t* src[kConcatMax];
  uint32_t off[kConcatMax + 1];   // first output column of input i; off[n] = W
};
void concat_last(uint32_t* dst, const ConcatLast& c, int64_t rows, hipStream_t st);
void fill(void* dst, int dt, double value, int64_t n, hipStream_t st);
void arange(void* dst, int dt, int64_t n, hipStream_t st);
void one_hot(const int32_t* idx, int64_t rows, int64_t depth, void* out, int dt, hipStream_t st);
// Stochastic ops: the seed lives in device memory (a per-step tensor input).
void dropout(const float* a, float* out, int64_t n, const int32_t* seed, uint32_t salt_const, double p,
             hipStream_t st);
void randn(float* out, int64_t n, const int32_t* seed, uint32_t salt_const, hipStream_t st);
void categorical(const float* a, int32_t* out, int64_t outer, int64_t D, const int32_t* seed, uint32_t salt_const,
                 hipStream_t st);

// ---- fused element-wise groups (k_fused.hip) ------------------------------------------
constexpr int kFusedRegs = 16;
constexpr int kFusedMaxInstr = 64;
// Operand access modes. With several elements per thread (vec 4), a strided operand's
// innermost stride decides how the thread's run of elements is read: FM_STRIDED_V one
// 128-bit load (innermost stride 1, 16-byte aligned), FM_STRIDED_B one load shared by
// the run (innermost stride 0), FM_STRIDED one load per element.
enum FusedMode { FM_CONTIG = 0, FM_SCALAR = 1, FM_STRIDED = 2, FM_STRIDED_V = 3, FM_STRIDED_B = 4 };
struct FusedInstr {
  int32_t op, dst, a, b, c;
  int32_t dt, ta, tb;             // result dtype (DT_F32 / DT_I32) and operand dtypes
  uint32_t salt;                  // dropout salt constant
  double imm, imm2;               // scalar operand; dropout p and 1/(1-p)
};
// A group program: registers 0..n_in-1 are the loaded operands, instructions write
// further registers, out_reg[] are stored. The header travels as a kernel argument; the
// instructions live in device memory (`code`) and are read with scalar loads.
// Each thread handles `vec` consecutive elements; the iteration space is `rank` merged
// dims (the innermost divided by vec) with 32-bit indices, so every tensor the group
// touches has fewer than 2^31 elements.
struct FusedProgram {
  int32_t n_in, n_out, n_instr, rank, any_strided, vec;
  // Row form when row_d > 0: the iteration space is rows x row_d, `rank` / div /
  // in_strides describe the merged row dims, in_inner the column stride, and out_row
  // marks per-row outputs.
  int32_t row_d;
  int32_t out_row[8];
  int32_t nregs;          // registers the program uses (LDS is sized from it)
  FastDiv div[kMaxRank];
  const void* in[kFusedMaxIn];
  int32_t in_dt[kFusedMaxIn], in_mode[kFusedMaxIn], in_inner[kFusedMaxIn];
  int32_t in_strides[kFusedMaxIn][kMaxRank];   // per dim of the iteration space (innermost x vec)
  void* out[kFusedMaxOut];
  int32_t out_dt[kFusedMaxOut], out_reg[kFusedMaxOut];
  const int32_t* seed;
  const FusedInstr* code;
};
// `n` = number of threads' runs (elements / vec), or of rows in the row form.
void fused(const FusedProgram& prog, int64_t n, hipStream_t st);

// ---- reductions / softmax (k_reduce.hip) --------------------------------------------
// Deterministic parallel sums with f64 accumulation: out[c] = f32(sum_r a[cell(c) +
// red(r)] / div) for c < ncells, r < nred. `cells` / `red` carry dims and element
// strides in s0. Used for sum_last / mean_last (red = last axis) and for the
// un-broadcast sums of autograd (sum_to_shape). `work` must hold
// sum_workspace_doubles(...) doubles of partials and `counters` sum_counters(...) zeroed
// counters of its own (a launch leaves them zero again).
int64_t sum_workspace_doubles(const Strided& cells, const Strided& red, int64_t ncells, int64_t nred);
int64_t sum_counters(const Strided& cells, const Strided& red, int64_t ncells, int64_t nred);
void reduce_sum(const float* a, float* out, const Strided& cells, const Strided& red, int64_t ncells, int64_t nred,
                double div, double* work, unsigned* counters, hipStream_t st);
// Column sums of [R, C] row-major operands (row stride rs), out[c] = f32(sum_r x / div)
// with x = a or the f32 product a * b, up to kColSumMax independent sums in one launch.
// `part` holds colsum_workspace_doubles(C, R, terms) doubles and `counters` colsum_counters(C, R, terms)
// zeroed counters per sum (left zero again), terms = 2 for a sum of products, else 1.
struct ColSum {
  const float* a;
  const float* b;
  float* out;
  int64_t C, R, rs, chunk;
  int nchunks, nx;
  int cpl;                // consecutive columns per lane (4 when C and rs allow, else 1)
  int aligned;            // cpl == 4 and every row start 16-byte aligned: 128-bit loads
  int blk0;               // first block of this sum in the launch (set by colsum_batch)
  double div;
  double scale;           // != 1: out = f32(f32(sum / div) * scale), a mul_scalar after the sum
  double* part;
  unsigned* counters;
  const double* pin;      // non-null: sum the f64 rows pin[r * rs + c] (GEMM epilogue partials) instead of a
};
constexpr int kColSumMax = 32;
// An embedding gradient of the scatter_scan_form run by the first `blocks` blocks of a
// column-sum launch (blocks = V * ceil(N / 512): one block per token and 512 columns), so
// its latency hides under the sums; idx null: none.
struct ColSumScatter {
  const int32_t* idx;
  const float* dy;
  float* out;
  int64_t rows, N;
  int V, blocks;
  // rows split into nwin windows of wrows: block (v, column block, window) sums its window,
  // the last of a (v, column block)'s windows adds the f64 partials part[v][window][c] in
  // window order (counter per (v, column block), left zero)
  int nwin;
  int64_t wrows;
  double* part;
  unsigned* counters;
};
// Row windows of the embedding gradient inside a column-sum launch (1: one block per token
// and column block walks every row), its partials (doubles) and counters.
int scatter_windows(int64_t rows, int64_t V, int64_t N);
int64_t scatter_workspace_doubles(int64_t rows, int64_t V, int64_t N);
int64_t scatter_counters(int64_t rows, int64_t V, int64_t N);
// Sum over the outer and inner axes of a contiguous [B, C, L] array (a convolution's bias
// gradient: images and spatial positions), out[c] = f32(sum over b and l), run by blocks
// of a column-sum launch after the scatter's: block (c, q) sums images q chunk .. in f64,
// and the last of channel c's nchunks blocks adds their partials in chunk order.
struct MidSum {
  const float* a;
  float* out;
  int64_t B, C, L, chunk;
  int nchunks, blk0;      // blk0: first block among the launch's MidSum blocks (set by colsum_batch)
  double* part;           // C * nchunks partials
  unsigned* counters;     // C counters, zero, left zero
};
constexpr int kMidSumMax = 2;
struct ColSumBatch {
  int n;
  ColSum s[kColSumMax];
  ColSumScatter sc;
  int nmid;
  MidSum m[kMidSumMax];
};
static_assert(sizeof(ColSumBatch) <= 4096, "column-sum batch fits the kernel argument space");
// `scale`: chunk-length multiple of the batch (colsum_batch_scale), the same at planning
// (workspace, counters) and at binding
ColSum colsum_desc(const float* a, const float* b, float* out, int64_t C, int64_t R, int64_t rs, double div,
                   double* part, unsigned* counters, int scale);
// The same sum over R rows of f64 partials (row stride C), as a term count of one.
ColSum colsum_desc_f64(const double* pin, float* out, int64_t C, int64_t R, double* part, unsigned* counters,
                       int scale);
int64_t colsum_workspace_doubles(int64_t C, int64_t R, int terms, int scale = 1);
int colsum_batch_scale(const int64_t* C, const int64_t* R, const int* terms, int n);
MidSum midsum_desc(const float* a, float* out, int64_t B, int64_t C, int64_t L, double* part, unsigned* counters);
int64_t midsum_workspace_doubles(int64_t B, int64_t C, int64_t L);
int64_t midsum_counters(int64_t B, int64_t C, int64_t L);
int64_t colsum_counters(int64_t C, int64_t R, int terms, int scale = 1);
void colsum_batch(const ColSumBatch& b, hipStream_t st);
void row_argmax(const float* a, int32_t* out, int64_t outer, int64_t D, hipStream_t st);
void log_softmax(const float* a, float* out, int64_t outer, int64_t D, hipStream_t st);
void softmax_causal(const float* a, float* out, int64_t mats, int64_t D, hipStream_t st);

// ---- fused causal attention (k_attention.hip) --------------------------------------
// Per (b, h): O = dropout(causal_softmax(f32(Q K^T * scale))) V, writing P (the softmax)
// and Pd (after dropout; null without dropout) as [B, H, T, T] contiguous. Q, V, O are
// [B, H, T, dh] and K [B, H, T, dh] (read as K^T) with unit stride along dh and the
// given element strides; all 16-byte aligned. Supported: dh = 64 with T = 64 or 128, and
// any T <= 64 with dh <= 64 (attention_supported).
struct AttnDesc {
  int B, H, T, dh;
  const float* q;
  int64_t sqb, sqh, sqi;
  const float* k;
  int64_t skb, skh, skj;
  const float* v;
  int64_t svb, svh, svj;
  float* o;
  int64_t sob, soh, soi;
  float* p;
  float* pd;
  int has_scale;
  double scale;
  int has_dropout;
  double drop_p, drop_scale;
  uint32_t salt;
  const int32_t* seed;
};
bool attention_supported(int64_t T, int64_t dh);
void attention_fwd(const AttnDesc& a, hipStream_t st);
// Backward of the same chain, given dO: dPd = dO V^T, dP = dropout(dPd) (forward mask),
// dS = f32(((dP - rowsum(dP * P)) * P) * scale), dQ = dS K, dK = dS^T Q, dV = Pd^T dO.
// dS is written to `ds` ([B, H, T, T]); dQ, dK, dV through their element strides
// (b, h, row, d), dQ and dV with unit d stride.
struct AttnBwdDesc {
  int B, H, T, dh;
  const float* dout;
  int64_t sob, soh, soi;
  const float* q;
  int64_t sqb, sqh, sqi;
  const float* k;
  int64_t skb, skh, skj;
  const float* v;
  int64_t svb, svh, svj;
  const float* p;
  const float* pd;
  float* ds;
  float* dq;
  int64_t sdqb, sdqh, sdqi;
  float* dk;
  int64_t sdkb, sdkh, sdkj, sdkd;
  float* dv;
  int64_t sdvb, sdvh, sdvj;
  int has_scale;
  double scale;
  int has_dropout;
  double drop_p, drop_scale;
  uint32_t salt;
  const int32_t* seed;
};
void attention_bwd(const AttnBwdDesc& a, hipStream_t st);

// ---- GEMM (k_gemm.hip; GemmDesc and the tile in gemm_dev.h) ----------------------------
// `work` must hold gemm_workspace_floats(d) floats (split-K partials).
int64_t gemm_workspace_floats(const GemmDesc& d);
void gemm(const GemmDesc& d, float* work, hipStream_t st);
// Grouped launch of independent GEMMs (whole-K 64 x 64 tiles, no split-K). Problems of one
// launch share a kind: gemm_group_kind(d) is 0..3, or -1 when d cannot run grouped.
// gemm_group_table fills the device image of the problem table (returns the offset of
// its tile-start array, sets the launch's block count and the tiling gemm_group takes:
// 1 for 32-k stages, two blocks per CU, when the launch has two or more tiles per CU and
// short K, else 0); the image must be copied to device memory and stay there while the
// launch can run.
int gemm_group_kind(const GemmDesc& d);
// A GEMM whose epilogue runs a fused element group (a kernel generated at run time): the
// tile configuration its plain launch would use, the group input that reads the product
// (h_in) and the product's row length N. gemm_epi_cfg fills the configuration, the launch
// arguments and the block count; false when d has no direct-to-LDS single-pass launch.
// Sum of products C = sum_s A_s B_s (n <= 4 terms with one shape and shared strides) as one
// launch; gemm_sum_ok tells whether the direct-to-LDS kernel takes the terms as given.
bool gemm_sum_ok(const GemmDesc* ds, int n);
void gemm_sum(const GemmDesc* ds, int n, hipStream_t st);
struct GemmEpiCfg {
  int bm, bn, bk, ns, nt, kg;
  bool ak, bkf;
  int64_t N;
  int h_in;
  bool store_c = false;   // the epilogue also stores the product itself to C
  bool cat = false;       // A is a concatenation along k (gemm_cat)
  int colsum_out = -1;    // output whose column partial sums the epilogue writes (GemmArgs::colsum)
  bool smallk = false;    // the small-K kernel (smallk_tile, bm rows of k padded to bk) instead of the tile
  bool gen = false;       // the element-wise tile (both operands one element per lane, partial k stages)
  bool tiny = false;      // the tiny kernel (tiny_tile, bm lanes per output; no column partials)
  bool skinny = false;    // the skinny kernel (skinny_tile, bm column tiles, bk: 16-byte A loads; no column partials)
};
// Rows of the f64 column partials an epilogue with colsum_out writes for this launch
// (tiles along M times the wavefronts along M of a tile).
int64_t gemm_epi_colsum_rows(const GemmEpiCfg& c, const gd::GemmArgs& g);
bool gemm_epi_cfg(const GemmDesc& d, GemmEpiCfg& c, gd::GemmArgs& g, int64_t& blocks);
// A product whose A operand is a concatenation along k of two row-major sources: k < k0
// from d.A (rows 16-byte aligned, k0 a multiple of 32), the rest from a1 (row stride lda1,
// any alignment); B rows contiguous, one batch. No workspace.
struct GemmCat {
  const float* a1;
  int64_t k0, lda1;
};
bool gemm_cat_ok(const GemmDesc& d, const GemmCat& c);
void gemm_cat(const GemmDesc& d, const GemmCat& c, hipStream_t st);
bool gemm_cat_epi_cfg(const GemmDesc& d, const GemmCat& c, GemmEpiCfg& cfg, gd::GemmArgs& g, int64_t& blocks);
// True when d on its own would run one pass of 64 x 64 tiles (the grouped tiling); the
// grouped launch's k-stage depth follows its own tile count, as a plain launch's does.
bool gemm_prefers_group(const GemmDesc& d);
size_t gemm_group_table(const GemmDesc* ds, int n, std::vector<unsigned char>& image, int64_t& blocks, int& tiling);
void gemm_group(const void* dev_image, size_t starts_off, int n, int64_t blocks, int kind, int tiling,
                hipStream_t st);

// Embedding pattern: out[r, :] = table[idx[r], :] (zero row when idx out of range).
void gather_rows(const int32_t* idx, int64_t rows, const float* table, int64_t V, int64_t N, float* out,
                 hipStream_t st);
// Embedding gradient: out[v, :] = sum over rows r with idx[r] == v of dy[r, :], in row
// order, f64 accumulation (V <= 8192); `work` must hold scatter_workspace_bytes(...)
// bytes, 256-byte aligned.
int64_t scatter_workspace_bytes(int64_t rows, int64_t V, int64_t N);
// The sort-free form (small V * rows): one launch, no workspace; the form a column-sum
// launch can run beside its sums (ColSumScatter).
bool scatter_scan_form(int64_t rows, int64_t V);
void scatter_rows(const int32_t* idx, int64_t rows, const float* dy, int64_t V, int64_t N, float* out, void* work,
                  hipStream_t st);

// ---- conv / pool (k_conv.hip) ---------------------------------------------------------
struct ConvDesc {
  int64_t B, Cin, H, W, Cout, CinPG, kH, kW, Ho, Wo, G, sH, sW, pH, pW;
};
void conv2d(const float* x, const float* w, float* y, const ConvDesc& c, hipStream_t st);
void conv2d_input_grad(const float* w, const float* dy, float* dx, const ConvDesc& c, hipStream_t st);
int64_t conv2d_weight_grad_workspace(const ConvDesc& c);
void conv2d_weight_grad(const float* x, const float* dy, float* dw, const ConvDesc& c, double* work, hipStream_t st);
// Implicit-GEMM convolutions on the matrix cores (k_conv_gemm.hip); f32 MFMA accumulation
// (GEMM tolerance against the f64 evaluator). conv_gemm_ok: every tensor indexable in 32
// bits. The weight gradient splits its batch reduction; `work` holds
// conv_gemm_workspace_bytes(c) bytes (0: none needed), at most kConvWorkBytes.
constexpr int64_t kConvWorkBytes = int64_t(12) << 20;
bool conv_gemm_ok(const ConvDesc& c);
int64_t conv_gemm_workspace_bytes(const ConvDesc& c);
// bias: store relu(y + bias[channel]) instead of y (the layer's bias + ReLU group; one
// group of channels). mask: store relu_grad(mask, dx) = mask > 0 ? dx : +0 instead of dx.
void conv2d_gemm(const float* x, const float* w, float* y, const ConvDesc& c, hipStream_t st,
                 const float* bias = nullptr);
void conv2d_input_grad_gemm(const float* w, const float* dy, float* dx, const ConvDesc& c, hipStream_t st,
                            const float* mask = nullptr);
void conv2d_weight_grad_gemm(const float* x, const float* dy, float* dw, const ConvDesc& c, float* work,
                             hipStream_t st);
struct PoolDesc { int64_t B, C, H, W, Ho, Wo, kH, kW, sH, sW, pH, pW; };
void max_pool(const float* x, float* y, const PoolDesc& p, hipStream_t st);
// relu: also apply relu_grad(x, .) with x the pool's input (the ReLU output it pools):
// dx = x > 0 ? dx : +0, in the same launch.
void max_pool_grad(const float* x, const float* dy, float* dx, const PoolDesc& p, hipStream_t st, bool relu = false);

// ---- optimizer (k_optim.hip) ----------------------------------------------------------
// One fused multi-tensor update (Adam / AdamW, or SGD with momentum, Nesterov and L2
// decay), in place on p and the optimizer state, with the gradient transforms of
// normalizeGrads and clipGradNorm applied to each gradient element on the fly.
// One launch unit: up to kAdamChunk consecutive elements of one parameter (pointers
// already offset to the chunk's first element).
constexpr int64_t kAdamChunk = 2048;
struct AdamChunk {
  float* p; float* m; float* v; const float* g;   // SGD: m = velocity (null: no momentum)
  const float* shrink_ptr;  // Adam: per-step decay shrink tensor, or null: use `shrink`
  double shrink;            // Adam: static decay shrink; SGD: weight decay (0: none)
  double mom;               // SGD: momentum (0: none)
  int64_t n;                // elements in the chunk, 1 .. kAdamChunk
  int gdiv, gmul;           // value indices: g = f32(g / vals[gdiv]) then f32(g * vals[gmul]); -1: none
  int flags;                // SGD: 1 Nesterov, 2 weight decay, 4 momentum
};
struct AdamHyper { double beta1, one_minus_beta1, beta2, one_minus_beta2, eps; };
// `chunks` is a device array of `nchunks` descriptors covering every parameter; `vals` the
// value array of the gradient-norm launches (null when no chunk transforms its gradient).
// Adam reads the f32 lrt at `lr`, SGD the f32 learning rate.
void adam_multi(const AdamChunk* chunks, int64_t nchunks, const float* lr, AdamHyper h, const float* vals,
                hipStream_t st);
void sgd_multi(const AdamChunk* chunks, int64_t nchunks, const float* lr, const float* vals, hipStream_t st);

// Gradient norms for clipGradNorm / normalizeGrads: per-tensor sums of squares, f32(x * x)
// summed in f64 and rounded to f32 once (the evaluator's mul + sum_last), then a scalar
// program over them (the reference's chained f32 adds, sqrt, add_scalar, div, min).
// Deterministic: chunk partials in a fixed order, a sum's chunk partials added in a fixed
// tree whichever block finishes it. The last block of a sum's chunks finishes that sum;
// the block finishing the last sum runs the program.
constexpr int64_t kNormChunk = 8192;   // gradient elements per block of a norm launch
struct SqChunk {
  const float* g;
  int64_t n;     // 1 .. kNormChunk
  int pre;       // value index dividing each element before squaring (normalised gradient), -1 none
  int slot;      // sum this chunk belongs to
};
enum ScalarOp { SI_CONST, SI_ADD, SI_SUB, SI_MUL, SI_DIV, SI_MIN, SI_MAX, SI_ADDK, SI_MULK, SI_SQRT };
struct ScalarInstr { int op, a, b, out; double k; };   // vals[out] = f32(vals[a] op vals[b] | k)
constexpr int kNormMaxVals = 2048;                     // value array bound (LDS of the finishing block)
struct NormLaunch {
  const SqChunk* chunks; int64_t nchunks;
  const int* slot_first;   // nslots + 1 chunk offsets: chunks of slot s are [first[s], first[s+1])
  const int* slot_val;     // value index receiving slot s's rounded sum
  int nslots;
  const ScalarInstr* prog; int nprog;
  float* vals; int nvals;
  double* part;            // nchunks partials (workspace)
  unsigned* counters;      // nslots + 1 launch-completion counters, left at zero
};
void grad_norms(const NormLaunch& a, hipStream_t st);

}  // namespace tgk
