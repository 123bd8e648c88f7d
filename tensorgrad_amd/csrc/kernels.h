// Host-side launch wrappers for the gfx950 kernels. Each wrapper enqueues one kernel on
// `st`; shapes arrive as plain integers (no torch types). All element storage is 4-byte:
// f32, or i32 for the `i32` and `bool` IR dtypes.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace tgk {

constexpr int kMaxRank = 8;

// dtype codes for element-wise operands
enum { DT_F32 = 0, DT_I32 = 1 };

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
void fill(void* dst, int dt, double value, int64_t n, hipStream_t st);
void arange(void* dst, int dt, int64_t n, hipStream_t st);
void one_hot(const int32_t* idx, int64_t rows, int64_t depth, void* out, int dt, hipStream_t st);
// Stochastic ops: the seed lives in device memory (a per-step tensor input).
void dropout(const float* a, float* out, int64_t n, const int32_t* seed, uint32_t salt_const, double p,
             hipStream_t st);
void randn(float* out, int64_t n, const int32_t* seed, uint32_t salt_const, hipStream_t st);
void categorical(const float* a, int32_t* out, int64_t outer, int64_t D, const int32_t* seed, uint32_t salt_const,
                 hipStream_t st);

// ---- reductions / softmax (k_reduce.hip) --------------------------------------------
// Deterministic parallel sums with f64 accumulation: out[c] = f32(sum_r a[cell(c) +
// red(r)] / div) for c < ncells, r < nred. `cells` / `red` carry dims and element
// strides in s0. Used for sum_last / mean_last (red = last axis) and for the
// un-broadcast sums of autograd (sum_to_shape). `work` must hold
// sum_workspace_doubles(...) doubles of partials.
int64_t sum_workspace_doubles(const Strided& cells, int64_t ncells, int64_t nred);
void reduce_sum(const float* a, float* out, const Strided& cells, const Strided& red, int64_t ncells, int64_t nred,
                double div, double* work, hipStream_t st);
void row_argmax(const float* a, int32_t* out, int64_t outer, int64_t D, hipStream_t st);
void log_softmax(const float* a, float* out, int64_t outer, int64_t D, hipStream_t st);
void softmax_causal(const float* a, float* out, int64_t mats, int64_t D, hipStream_t st);

// ---- GEMM (k_gemm.hip) --------------------------------------------------------------
// C[z][m][n] = sum_k A[z][m][k] * B[z][k][n], f32 MFMA, f32 accumulate.
// Batch index z decomposes as (z / bdiv, z % bdiv) with two strides per operand, so a
// permuted 4-d view [B, H, T, d] is read in place.
struct GemmDesc {
  int64_t M, N, K, batch, bdiv;
  const float* A; int64_t sAz0, sAz1, sAm, sAk;
  const float* B; int64_t sBz0, sBz1, sBk, sBn;
  float* C; int64_t sCz0, sCz1, sCm, sCn;
};
// `work` must hold gemm_workspace_floats(d) floats (split-K partials).
int64_t gemm_workspace_floats(const GemmDesc& d);
void gemm(const GemmDesc& d, float* work, hipStream_t st);

// Embedding pattern: out[r, :] = table[idx[r], :] (zero row when idx out of range).
void gather_rows(const int32_t* idx, int64_t rows, const float* table, int64_t V, int64_t N, float* out,
                 hipStream_t st);
// Embedding gradient: out[v, :] = sum over rows r with idx[r] == v of dy[r, :], in row
// order, f64 accumulation; needs `perm` (rows ints) and `offs` (2V + 1 ints) scratch.
void scatter_rows(const int32_t* idx, int64_t rows, const float* dy, int64_t V, int64_t N, float* out,
                  int32_t* perm, int32_t* offs, hipStream_t st);

// ---- conv / pool (k_conv.hip) ---------------------------------------------------------
struct ConvDesc {
  int64_t B, Cin, H, W, Cout, CinPG, kH, kW, Ho, Wo, G, sH, sW, pH, pW;
};
void conv2d(const float* x, const float* w, float* y, const ConvDesc& c, hipStream_t st);
void conv2d_input_grad(const float* w, const float* dy, float* dx, const ConvDesc& c, hipStream_t st);
int64_t conv2d_weight_grad_workspace(const ConvDesc& c);
void conv2d_weight_grad(const float* x, const float* dy, float* dw, const ConvDesc& c, double* work, hipStream_t st);
struct PoolDesc { int64_t B, C, H, W, Ho, Wo, kH, kW, sH, sW, pH, pW; };
void max_pool(const float* x, float* y, const PoolDesc& p, hipStream_t st);
void max_pool_grad(const float* x, const float* dy, float* dx, const PoolDesc& p, hipStream_t st);

// ---- optimizer (k_optim.hip) ----------------------------------------------------------
// One fused multi-tensor Adam/AdamW update, in place on p, m, v.
struct AdamTensor {
  float* p; float* m; float* v; const float* g;
  int64_t n;
  double shrink;          // literal decayShrink (used when shrink_ptr is null)
  const float* shrink_ptr;
};
struct AdamHyper { double beta1, one_minus_beta1, beta2, one_minus_beta2, eps; };
// `tensors` is a device array of `count` AdamTensor; `chunks` maps blocks to tensors.
void adam_multi(const AdamTensor* tensors, int count, const int64_t* chunk_tensor, const int64_t* chunk_start,
                int64_t nchunks, const float* lrt, AdamHyper h, hipStream_t st);

}  // namespace tgk
