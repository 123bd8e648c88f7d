// CPU ORACLE — test infrastructure only. Restates the reference's CPU IR evaluator
// (test/_eval.ts) op by op, extended with the Adam convention and the worker's per-step
// scalar logic, so that the GPU backend can be checked against it on identical inputs.
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
// library; the product path never does.
//
// Numeric conventions kept from the reference evaluator (they fix the bit patterns):
//  * every tensor is stored as f32 (Float32Array) or i32 (Int32Array) between ops;
//  * element-wise ops compute in f64 on the f32 operands and round once on store
//    (_eval.ts:133-203);
//  * matmul / conv / reductions / softmaxes accumulate in f64 in the reference's loop
//    order (_eval.ts:206-236, 271-314, 361-405, 619-715);
//  * sum_to_shape accumulates into the f32 output array in source-flat order
//    (_eval.ts:492-523);
//  * dropout / categorical hash with an f64 multiply before `>>> 0` (_eval.ts:568-574,
//    595-603); randn uses Math.imul (_eval.ts:544-553);
//  * Adam (the reference evaluator throws on it, _eval.ts:611-614): m', v', p' computed
//    in f64 from f32 operands with the f64 constants beta1, 1-beta1, beta2, 1-beta2, eps
//    and the literal decayShrink, each output rounded to f32 once; formula of
//    src/codegen.ts:854, 873, 899.
// Two switches for the parity fixtures only (off by default) measure how far other valid
// roundings drift: orc_set_matmul_f32 makes matmuls accumulate in f32, orc_set_sum_f64
// makes sum_to_shape accumulate in f64.
// Per-element loops are parallelised over output elements with OpenMP; each element's
// own accumulation order is unchanged, so results are bit-identical for any thread count.
//
// Compiled with -ffp-contract=off: no fused multiply-add may change a rounding.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <set>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "jsonv.hpp"

namespace orc {

static thread_local std::string g_err;

using Shape = std::vector<int64_t>;

static int64_t numel(const Shape& s) { int64_t n = 1; for (auto d : s) n *= d; return n; }

// C[z] = A[z] * B[z or 0] with f64 running sums in increasing k for every output: the same
// sequence of roundings as the evaluator's per-output loop, so bit-identical to it. The
// loops are blocked (4 rows x 256 columns of running sums, k outermost inside a block) so
// B is read row by row; B's rows are widened to f64 once per block column. Built for AVX2
// and baseline x86-64 (chosen at load time); -ffp-contract=off keeps mul and add separate.
__attribute__((target_clones("avx2", "default")))
static void matmul_block(const float* __restrict__ A, const double* __restrict__ Bd, float* __restrict__ C, int64_t M,
                         int64_t K, int64_t N, int64_t m0, int64_t mr, int64_t n0, int64_t nn) {
  constexpr int64_t MR = 4, NB = 256;
  double acc[MR][NB];
  for (int64_t r = 0; r < mr; ++r)
    for (int64_t j = 0; j < nn; ++j) acc[r][j] = 0.0;
  for (int64_t kk = 0; kk < K; ++kk) {
    const double* brow = Bd + kk * nn;
    for (int64_t r = 0; r < mr; ++r) {
      const double av = (double)A[(m0 + r) * K + kk];
      double* __restrict__ ar = acc[r];
      for (int64_t j = 0; j < nn; ++j) ar[j] += av * brow[j];
    }
  }
  for (int64_t r = 0; r < mr; ++r)
    for (int64_t j = 0; j < nn; ++j) C[(m0 + r) * N + n0 + j] = (float)acc[r][j];
}

// The f32 twin of the parity fixtures (orc_set_matmul_f32): the same loop with f32
// running sums (each product rounded to f32, then added in f32, increasing k), the
// accumulation an f32 GPU kernel uses; off unless a fixture script turns it on.
static bool g_matmul_f32 = false;
// The f64-sum twin (orc_set_sum_f64): sum_to_shape accumulates in f64 and rounds once, as
// the GPU's column sums do; off unless a fixture script turns it on.
static bool g_sum_f64 = false;

__attribute__((target_clones("avx2", "default")))
static void matmul_block_f32(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int64_t M,
                             int64_t K, int64_t N, int64_t m0, int64_t mr, int64_t n0, int64_t nn) {
  constexpr int64_t MR = 4, NB = 256;
  float acc[MR][NB];
  for (int64_t r = 0; r < mr; ++r)
    for (int64_t j = 0; j < nn; ++j) acc[r][j] = 0.0f;
  for (int64_t kk = 0; kk < K; ++kk) {
    const float* brow = B + kk * N + n0;
    for (int64_t r = 0; r < mr; ++r) {
      const float av = A[(m0 + r) * K + kk];
      float* __restrict__ ar = acc[r];
      for (int64_t j = 0; j < nn; ++j) ar[j] += av * brow[j];
    }
  }
  for (int64_t r = 0; r < mr; ++r)
    for (int64_t j = 0; j < nn; ++j) C[(m0 + r) * N + n0 + j] = acc[r][j];
}

static void matmul_f64(const float* A, const float* B, float* C, int64_t batch, int64_t M, int64_t K, int64_t N,
                       bool batched) {
  constexpr int64_t MR = 4, NB = 256;
  if (g_matmul_f32) {
    const int64_t mblocks = (M + MR - 1) / MR, nblocks = (N + NB - 1) / NB;
    for (int64_t bi = 0; bi < batch; ++bi) {
      const float* Bb = B + (batched ? bi * K * N : 0);
      for (int64_t nbk = 0; nbk < nblocks; ++nbk) {
        const int64_t n0 = nbk * NB, nn = std::min(NB, N - n0);
#pragma omp parallel for schedule(static)
        for (int64_t mb = 0; mb < mblocks; ++mb)
          matmul_block_f32(A + bi * M * K, Bb, C + bi * M * N, M, K, N, mb * MR, std::min(MR, M - mb * MR), n0, nn);
      }
    }
    return;
  }
  const int64_t mblocks = (M + MR - 1) / MR, nblocks = (N + NB - 1) / NB;
  for (int64_t bi = 0; bi < batch; ++bi) {
    const float* Bb = B + (batched ? bi * K * N : 0);
    for (int64_t nbk = 0; nbk < nblocks; ++nbk) {
      const int64_t n0 = nbk * NB, nn = std::min(NB, N - n0);
      std::vector<double> Bd((size_t)(K * nn));
      for (int64_t kk = 0; kk < K; ++kk)
        for (int64_t j = 0; j < nn; ++j) Bd[kk * nn + j] = (double)Bb[kk * N + n0 + j];
#pragma omp parallel for schedule(static)
      for (int64_t mb = 0; mb < mblocks; ++mb)
        matmul_block(A + bi * M * K, Bd.data(), C + bi * M * N, M, K, N, mb * MR, std::min(MR, M - mb * MR), n0, nn);
    }
  }
}


enum Dt { F32, I32, BOOL };
static Dt parse_dt(const std::string& s) {
  if (s == "f32") return F32;
  if (s == "i32") return I32;
  if (s == "bool") return BOOL;
  throw std::runtime_error("oracle: bad dtype " + s);
}

// A value: 4-byte elements, interpreted per dtype.
struct Val {
  Dt dt = F32;
  std::vector<uint32_t> raw;
  float* f() { return reinterpret_cast<float*>(raw.data()); }
  int32_t* i() { return reinterpret_cast<int32_t*>(raw.data()); }
  const float* f() const { return reinterpret_cast<const float*>(raw.data()); }
  const int32_t* i() const { return reinterpret_cast<const int32_t*>(raw.data()); }
  size_t n() const { return raw.size(); }
  // Numeric value of element k as a JS number (f64).
  double num(size_t k) const { return dt == F32 ? (double)f()[k] : (double)i()[k]; }
};

// JS ToInt32 of an f64 (used when an op stores into an Int32Array).
static int32_t to_int32(double x) {
  if (!std::isfinite(x)) return 0;
  double t = std::trunc(x);
  double m = std::fmod(t, 4294967296.0);
  if (m < 0) m += 4294967296.0;
  uint32_t u = (uint32_t)m;
  return (int32_t)u;
}

static void store(Val& v, size_t k, double x) {
  if (v.dt == F32) v.f()[k] = (float)x;
  else v.i()[k] = to_int32(x);
}

static Val make(Dt dt, int64_t n) { Val v; v.dt = dt == BOOL ? I32 : dt; v.raw.assign((size_t)n, 0u); return v; }

static std::vector<int64_t> strides_of(const Shape& s) {
  std::vector<int64_t> st(s.size(), 1);
  for (int i = (int)s.size() - 2; i >= 0; --i) st[i] = st[i + 1] * s[i + 1];
  return st;
}

// Right-aligned broadcast index (_eval.ts:49-70).
// Source shape equal to the trailing dims of the output (after dropping leading 1s): its
// element for output index i is i % numel(src) (what bidx computes, without the loop).
static bool trailing(const Shape& out, const Shape& src) {
  size_t s0 = 0;
  while (s0 < src.size() && src[s0] == 1) ++s0;
  const size_t n = src.size() - s0;
  if (n > out.size()) return false;
  for (size_t q = 0; q < n; ++q)
    if (src[s0 + q] != out[out.size() - n + q]) return false;
  return true;
}

static int64_t bidx(int64_t outIdx, const Shape& out, const Shape& src) {
  int64_t rankDiff = (int64_t)out.size() - (int64_t)src.size();
  int64_t aIdx = 0, aStride = 1, rem = outIdx;
  for (int64_t d = (int64_t)out.size() - 1; d >= 0; --d) {
    int64_t od = out[d];
    int64_t coord = rem % od;
    rem /= od;
    int64_t sa = d - rankDiff;
    if (sa >= 0) {
      int64_t sd = src[sa];
      if (sd != 1) aIdx += coord * aStride;
      aStride *= sd;
    }
  }
  return aIdx;
}

// JS Math.max / Math.min semantics (NaN-propagating, +0 > -0).
static double js_max(double a, double b) {
  if (std::isnan(a) || std::isnan(b)) return std::numeric_limits<double>::quiet_NaN();
  if (a == 0 && b == 0) return (std::signbit(a) && std::signbit(b)) ? -0.0 : 0.0;
  return a > b ? a : b;
}
static double js_min(double a, double b) {
  if (std::isnan(a) || std::isnan(b)) return std::numeric_limits<double>::quiet_NaN();
  if (a == 0 && b == 0) return (std::signbit(a) || std::signbit(b)) ? -0.0 : 0.0;
  return a < b ? a : b;
}
static double js_sign(double x) {
  if (std::isnan(x)) return x;
  if (x > 0) return 1;
  if (x < 0) return -1;
  return x;  // keeps the sign of zero
}

// JS `>>> 0` of an f64 holding an integer value (ToUint32).
static uint32_t to_uint32(double x) {
  double m = std::fmod(std::trunc(x), 4294967296.0);
  if (m < 0) m += 4294967296.0;
  return (uint32_t)m;
}

// ToUint32 of a non-negative integral f64 below 2^64: its value modulo 2^32.
static inline uint32_t to_uint32_nonneg(double x) { return (uint32_t)(uint64_t)x; }

// The dropout / categorical hash: PCG-RXS-M-XS evaluated the way _eval.ts:568-571 does,
// with the two multiplies as IEEE f64 products (rounded above 2^53) before ToUint32.
static uint32_t pcg_f64(uint32_t seed, uint32_t saltConst, uint32_t idx) {
  uint32_t h = seed ^ saltConst ^ idx;
  // both products and the sum are non-negative integers below 2^63
  volatile double prod = (double)h * 747796405.0;
  h = to_uint32_nonneg(prod + 2891336453.0);
  uint32_t x = h ^ (h >> ((h >> 28) + 4));
  volatile double prod2 = (double)x * 277803737.0;
  h = to_uint32_nonneg(prod2);
  h = h ^ (h >> 22);
  return h;
}

// The randn hash (_eval.ts:544-550) with Math.imul (wrapping u32 multiplies).
static void pcg_imul2(uint32_t seed, uint32_t saltConst, uint32_t idx, uint32_t& h1o, uint32_t& h2o) {
  uint32_t h1 = seed ^ saltConst ^ idx;
  h1 = h1 * 747796405u + 2891336453u;
  h1 = (h1 ^ (h1 >> ((h1 >> 28) + 4))) * 277803737u;
  h1 = h1 ^ (h1 >> 22);
  uint32_t h2 = h1 * 747796405u + 2891336453u;
  h2 = (h2 ^ (h2 >> ((h2 >> 28) + 4))) * 277803737u;
  h2 = h2 ^ (h2 >> 22);
  h1o = h1; h2o = h2;
}

static uint32_t salt_const(int64_t salt) {
  // (salt * 0x9E3779B1) >>> 0 with an f64 product (exact for salt < 2^21).
  double p = (double)salt * 2654435761.0;
  return to_uint32(p);
}

struct TensorInfo { Shape shape; Dt dt; };

struct LRSched;  // forward

// ---- learning-rate schedules (src/lr.ts:69-112) ----------------------------------------
static double resolve_lr(const JV& s, double step) {
  if (s.t == JV::NUM) return s.n;
  const std::string& k = s["kind"].str();
  const JV* ss = s.find("startStep");
  double start = (ss && !ss->is_null()) ? ss->n : 0;
  double st = std::max(1.0, step - start);
  if (k == "linear") {
    double f = std::min(st / s["steps"].num(), 1.0);
    return s["peak"].num() + (s["final"].num() - s["peak"].num()) * f;
  }
  if (k == "cosineAnnealing") {
    double f = std::min(st / s["steps"].num(), 1.0);
    return s["final"].num() + 0.5 * (s["peak"].num() - s["final"].num()) * (1 + std::cos(M_PI * f));
  }
  if (k == "warmup") {
    if (st <= s["steps"].num()) return s["peak"].num() * (st / s["steps"].num());
    return resolve_lr(s["after"], st - s["steps"].num());
  }
  if (k == "staircase") {
    double kk = std::floor((st - 1) / s["every"].num());
    return s["peak"].num() * std::pow(s["gamma"].num(), kk);
  }
  if (k == "multiStep") {
    double kk = 0;
    for (auto& m : s["milestones"].a) if (st >= m.n) kk += 1;
    return s["peak"].num() * std::pow(s["gamma"].num(), kk);
  }
  throw std::runtime_error("oracle: unknown lr kind " + k);
}

class Oracle {
 public:
  explicit Oracle(const char* wire) : doc_(parse_json(wire)) {
    const JV& g = doc_["graph"];
    for (auto& t : g["tensors"].a) {
      TensorInfo ti;
      for (auto& d : t["shape"].a) ti.shape.push_back(d.i64());
      ti.dt = parse_dt(t["dtype"].str());
      tinfo_.push_back(ti);
    }
    for (auto& op : g["ops"].a) ops_.push_back(&op);
    for (auto& o : g["outputs"].a) outputs_.push_back(o.i32());
    for (auto& c : g["captures"].o) captures_[c.first] = c.second.i32();
    for (auto* op : ops_) {
      const std::string& k = (*op)["kind"].str();
      int out = (*op)["out"].i32();
      if (k == "param_input") { params_.push_back((*op)["name"].str()); param_tid_[(*op)["name"].str()] = out; }
      if (k == "state_input") {
        std::string nm = (*op)["name"].str();
        state_tid_[nm] = out;
        Val v = make(tinfo_[out].dt, numel(tinfo_[out].shape));
        double iv = (*op)["initValue"].num();
        if (iv != 0 && tinfo_[out].dt == F32) for (size_t j = 0; j < v.n(); ++j) v.f()[j] = (float)iv;
        home_[nm] = v;
      }
      if (k == "tensor_input" && (*op)["name"].str() == "__prngSeed") uses_prng_ = true;
    }
    for (auto& p : params_) home_[p] = make(tinfo_[param_tid_[p]].dt, numel(tinfo_[param_tid_[p]].shape));
    const JV* wb = doc_.find("writebacks");
    if (wb) for (auto& w : wb->a) writebacks_.push_back({w["source"].i32(), w["destName"].str()});
    const JV* opt = doc_.find("optimizer");
    if (opt && !opt->is_null()) { opt_kind_ = (*opt)["kind"].str(); opt_cfg_ = &(*opt)["config"]; lr_ = (*opt_cfg_)["lr"]; }
  }

  const std::vector<std::string>& params() const { return params_; }
  Val& home(const std::string& name) {
    auto it = home_.find(name);
    if (it == home_.end()) throw std::runtime_error("oracle: unknown param/state '" + name + "'");
    return it->second;
  }
  int64_t home_numel(const std::string& name) { return (int64_t)home(name).n(); }

  // setLR (worker.ts:304-319): the new schedule is rebased so its step 1 is t + 1
  // (lr.ts:108-112) unless it carries an explicit startStep.
  void set_lr(const char* json) {
    lr_store_ = parse_json(json);
    if (lr_store_.t == JV::OBJ) {
      const JV* ss = lr_store_.find("startStep");
      if (!ss || ss->is_null()) {
        JV v; v.t = JV::NUM; v.n = (double)t_;
        bool set = false;
        for (auto& kv : lr_store_.o) if (kv.first == "startStep") { kv.second = v; set = true; }
        if (!set) lr_store_.o.emplace_back("startStep", v);
      }
    }
    lr_ = lr_store_;
    lr_overridden_ = true;
  }
  void reset_optimizer() {
    for (auto& kv : state_tid_) std::fill(home_[kv.first].raw.begin(), home_[kv.first].raw.end(), 0u);
    t_ = 0;
  }

  // One training step (worker.ts:187-240): bump t, inject lrt / decayShrink / lr and the
  // PRNG seed, evaluate every op, apply writebacks. Returns the loss.
  double step(const std::map<std::string, Val>& user_inputs) {
    std::map<std::string, Val> inputs = user_inputs;
    if (opt_cfg_) {
      ++t_;
      const JV& c = *opt_cfg_;
      double lrNow = resolve_lr(lr_, (double)t_);
      if (opt_kind_ == "adam") {
        double lrt = lrNow * std::sqrt(1 - std::pow(c["beta2"].num(), (double)t_)) / (1 - std::pow(c["beta1"].num(), (double)t_));
        Val v = make(F32, 1); v.f()[0] = (float)lrt;
        inputs[c["lrtInputName"].str()] = v;
        const JV& dn = c["decayShrinkInputName"];
        if (!dn.is_null()) {
          Val d = make(F32, 1); d.f()[0] = (float)(1 - lrNow * c["weightDecay"].num());
          inputs[dn.str()] = d;
        }
      } else {
        Val v = make(F32, 1); v.f()[0] = (float)lrNow;
        inputs[c["lrInputName"].str()] = v;
      }
    }
    inject_seed(inputs);
    eval(inputs, true);
    double loss = vals_.at(outputs_[0]).num(0);
    // Writebacks: every source is computed from pre-step values, so apply after eval.
    std::vector<std::pair<std::string, Val>> staged;
    for (auto& w : writebacks_) staged.emplace_back(w.second, vals_.at(w.first));
    for (auto& s : staged) {
      Val& h = home(s.first);
      if (h.n() != s.second.n()) throw std::runtime_error("oracle: writeback size mismatch for " + s.first);
      h.raw = s.second.raw;
    }
    return loss;
  }

  // Forward-only evaluation (worker.ts:242-260): seed injected, no optimizer scalars.
  void run(const std::map<std::string, Val>& user_inputs) {
    std::map<std::string, Val> inputs = user_inputs;
    inject_seed(inputs);
    eval(inputs, false);
  }

  const Val& value(int tid) const {
    auto it = vals_.find(tid);
    if (it == vals_.end()) throw std::runtime_error("oracle: tensor #" + std::to_string(tid) + " not retained");
    return it->second;
  }
  int output_tid() const { return outputs_.at(0); }
  const TensorInfo& info(int tid) const { return tinfo_.at(tid); }
  void retain_all(bool on) { retain_all_ = on; }

 private:
  JV doc_;
  JV lr_store_;
  JV lr_;
  bool lr_overridden_ = false;
  std::vector<TensorInfo> tinfo_;
  std::vector<const JV*> ops_;
  std::vector<int> outputs_;
  std::map<std::string, int> captures_;
  std::vector<std::string> params_;
  std::map<std::string, int> param_tid_, state_tid_;
  std::map<std::string, Val> home_;
  std::vector<std::pair<int, std::string>> writebacks_;
  std::string opt_kind_;
  const JV* opt_cfg_ = nullptr;
  long long t_ = 0;
  bool uses_prng_ = false;
  long long prng_counter_ = 0;
  bool retain_all_ = false;
  std::unordered_map<int, Val> vals_;

  // The worker always injects the per-graph counter (worker.ts:208-214). A test may
  // instead bind `__prngSeed` explicitly, as the reference's FD harness does
  // (test/grad.ts:78-81); an explicit seed is then used and the counter left alone.
  void inject_seed(std::map<std::string, Val>& inputs) {
    if (!uses_prng_ || inputs.count("__prngSeed")) return;
    ++prng_counter_;
    Val v = make(I32, 1); v.i()[0] = (int32_t)(uint32_t)prng_counter_;
    inputs["__prngSeed"] = v;
  }

  void eval(const std::map<std::string, Val>& inputs, bool training) {
    (void)training;
    vals_.clear();
    // Free intermediates after their last reader unless they must be kept.
    std::vector<int> last_use(tinfo_.size(), -1);
    for (size_t i = 0; i < ops_.size(); ++i) for (int id : op_inputs(*ops_[i])) last_use[id] = (int)i;
    std::set<int> keep(outputs_.begin(), outputs_.end());
    for (auto& c : captures_) keep.insert(c.second);
    for (auto& w : writebacks_) keep.insert(w.first);
    // ORC_PROFILE=1 in the environment prints the time spent per op kind (to stderr).
    static const bool prof = std::getenv("ORC_PROFILE") != nullptr;
    std::map<std::string, double> tk;
    for (size_t i = 0; i < ops_.size(); ++i) {
      const JV& op = *ops_[i];
      int out = op["out"].i32();
      const double t0 = prof ? omp_get_wtime() : 0.0;
      const std::string& kind = op["kind"].str();
      const JV* src = op.find("a");
      if ((kind == "reshape" || kind == "stop_gradient") && !retain_all_ && src && last_use[src->i32()] == (int)i &&
          !keep.count(src->i32()) && vals_.count(src->i32())) {
        // the input dies here: hand its storage over instead of copying it
        Val v = std::move(vals_[src->i32()]);
        vals_.erase(src->i32());
        const Dt dt = tinfo_[out].dt;
        v.dt = dt == BOOL ? I32 : dt;
        vals_[out] = std::move(v);
      } else {
        vals_[out] = eval_op(op, inputs);
      }
      if (prof) tk[op["kind"].str()] += omp_get_wtime() - t0;
      if (!retain_all_) {
        for (int id : op_inputs(op)) {
          if (last_use[id] == (int)i && !keep.count(id)) vals_.erase(id);
        }
      }
    }
    if (prof)
      for (auto& kv : tk) fprintf(stderr, "oracle %-22s %8.3f s\n", kv.first.c_str(), kv.second);
  }

  static std::vector<int> op_inputs(const JV& op) {
    static const std::map<std::string, std::vector<std::string>> F = {
        {"randn", {"seed"}}, {"dropout", {"a", "seed"}}, {"categorical_last", {"a", "seed"}},
        {"one_hot", {"indices"}}, {"where", {"cond", "a", "b"}}, {"relu_grad", {"x", "dy"}},
        {"adam_update_m", {"m", "g"}}, {"adam_update_v", {"v", "g"}},
        {"adam_update_p", {"p", "mNew", "vNew", "lrt", "decayShrinkTensor"}},
        {"conv2d", {"input", "weight"}}, {"conv2d_input_grad", {"weight", "dy"}},
        {"conv2d_weight_grad", {"input", "dy"}}, {"max_pool_2d", {"input"}}, {"max_pool_2d_grad", {"input", "dy"}},
    };
    const std::string& k = op["kind"].str();
    std::vector<int> ids;
    if (k == "concat") { for (auto& x : op["inputs"].a) ids.push_back(x.i32()); return ids; }
    auto it = F.find(k);
    if (it != F.end()) {
      for (auto& f : it->second) { const JV& v = op[f]; if (!v.is_null()) ids.push_back(v.i32()); }
      return ids;
    }
    if (op.find("b") && op.find("a")) { ids.push_back(op["a"].i32()); ids.push_back(op["b"].i32()); return ids; }
    if (op.find("a")) ids.push_back(op["a"].i32());
    return ids;
  }

  const Val& V(int id) const {
    auto it = vals_.find(id);
    if (it == vals_.end()) throw std::runtime_error("oracle: value #" + std::to_string(id) + " missing");
    return it->second;
  }
  const Shape& SH(int id) const { return tinfo_.at(id).shape; }

  Val eval_op(const JV& op, const std::map<std::string, Val>& inputs);
};

Val Oracle::eval_op(const JV& op, const std::map<std::string, Val>& inputs) {
  const std::string& k = op["kind"].str();
  int out = op["out"].i32();
  const Shape& shape = tinfo_[out].shape;
  Dt dt = tinfo_[out].dt;
  const int64_t total = numel(shape);

  if (k == "param_input") return home(op["name"].str());
  if (k == "tensor_input") {
    auto it = inputs.find(op["name"].str());
    if (it == inputs.end()) throw std::runtime_error("eval: missing input '" + op["name"].str() + "'");
    if ((int64_t)it->second.n() != total) throw std::runtime_error("eval: input '" + op["name"].str() + "' has wrong size");
    Val v = it->second; v.dt = dt == BOOL ? I32 : dt;
    return v;
  }
  if (k == "state_input") {
    auto it = inputs.find(op["name"].str());
    if (it != inputs.end()) return it->second;
    return home(op["name"].str());
  }
  if (k == "const_scalar") { Val v = make(dt, 1); store(v, 0, op["value"].num()); return v; }
  if (k == "const_fill") {
    Val v = make(dt, total);
    double x = op["value"].num();
    if (x != 0) for (int64_t i = 0; i < total; ++i) store(v, i, x);
    return v;
  }
  if (k == "arange") { Val v = make(dt, op["n"].i64()); for (int64_t i = 0; i < op["n"].i64(); ++i) store(v, i, (double)i); return v; }

  if (k == "add" || k == "sub" || k == "mul" || k == "div" || k == "min" || k == "max") {
    const Val& a = V(op["a"].i32()); const Val& b = V(op["b"].i32());
    const Shape& as = SH(op["a"].i32()); const Shape& bs = SH(op["b"].i32());
    Val o = make(dt, total);
    int which = k == "add" ? 0 : k == "sub" ? 1 : k == "mul" ? 2 : k == "div" ? 3 : k == "min" ? 4 : 5;
    const bool ta = trailing(shape, as), tb = trailing(shape, bs);
    const int64_t na = std::max<int64_t>(1, numel(as)), nb = std::max<int64_t>(1, numel(bs));
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; ++i) {
      double x = a.num(ta ? i % na : bidx(i, shape, as)), y = b.num(tb ? i % nb : bidx(i, shape, bs));
      double r;
      switch (which) {
        case 0: r = x + y; break;
        case 1: r = x - y; break;
        case 2: r = x * y; break;
        case 3: r = x / y; break;
        case 4: r = js_min(x, y); break;
        default: r = js_max(x, y);
      }
      store(o, i, r);
    }
    return o;
  }
  if (k == "mul_scalar" || k == "add_scalar") {
    const Val& a = V(op["a"].i32());
    double s = op["scalar"].num();
    Val o = make(F32, total);
    bool mulk = k == "mul_scalar";
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; ++i) o.f()[i] = (float)(mulk ? a.num(i) * s : a.num(i) + s);
    return o;
  }
  static const std::set<std::string> unary = {"sqrt", "rsqrt", "log", "exp", "relu", "neg", "abs", "tanh",
                                              "sigmoid", "erf", "sin", "cos"};
  if (unary.count(k)) {
    const Val& a = V(op["a"].i32());
    Val o = make(F32, (int64_t)a.n());
    int w = k == "sqrt" ? 0 : k == "rsqrt" ? 1 : k == "log" ? 2 : k == "exp" ? 3 : k == "relu" ? 4 : k == "neg" ? 5
          : k == "abs" ? 6 : k == "tanh" ? 7 : k == "sigmoid" ? 8 : k == "erf" ? 9 : k == "sin" ? 10 : 11;
    const int64_t n = (int64_t)a.n();
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
      double x = a.num(i), r;
      switch (w) {
        case 0: r = std::sqrt(x); break;
        case 1: r = 1 / std::sqrt(x); break;
        case 2: r = std::log(x); break;
        case 3: r = std::exp(x); break;
        case 4: r = js_max(x, 0); break;
        case 5: r = -x; break;
        case 6: r = std::fabs(x); break;
        case 7: r = std::tanh(x); break;
        case 8: r = 0.5 + 0.5 * std::tanh(0.5 * x); break;
        case 9: {  // A&S 7.1.26 (_eval.ts:193-198)
          double s = js_sign(x), ax = std::fabs(x);
          double t = 1 / (1 + 0.3275911 * ax);
          double p = t * (0.254829592 + t * (-0.284496736 + t * (1.421413741 + t * (-1.453152027 + t * 1.061405429))));
          r = s * (1 - p * std::exp(-ax * ax));
          break;
        }
        case 10: r = std::sin(x); break;
        default: r = std::cos(x);
      }
      o.f()[i] = (float)r;
    }
    return o;
  }
  if (k == "mean_last" || k == "sum_last") {
    const Val& a = V(op["a"].i32());
    const Shape& as = SH(op["a"].i32());
    int64_t D = as.back(), outer = numel(as) / D;
    Val o = make(F32, outer);
    double div = k == "mean_last" ? (double)D : 1.0;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < outer; ++i) {
      double s = 0;
      for (int64_t j = 0; j < D; ++j) s += a.num(i * D + j);
      o.f()[i] = (float)(s / div);
    }
    return o;
  }
  if (k == "argmax_last") {
    const Val& a = V(op["a"].i32());
    const Shape& as = SH(op["a"].i32());
    int64_t D = as.back(), outer = numel(as) / D;
    Val o = make(I32, outer);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < outer; ++i) {
      int64_t best = 0; double bv = a.num(i * D);
      for (int64_t j = 1; j < D; ++j) { double x = a.num(i * D + j); if (x > bv) { bv = x; best = j; } }
      o.i()[i] = (int32_t)best;
    }
    return o;
  }
  if (k == "reshape" || k == "stop_gradient") { Val v = V(op["a"].i32()); v.dt = dt == BOOL ? I32 : dt; return v; }
  if (k == "permute") {
    const Val& a = V(op["a"].i32());
    const Shape& as = SH(op["a"].i32());
    auto aStr = strides_of(as), oStr = strides_of(shape);
    std::vector<int64_t> perm;
    for (auto& p : op["perm"].a) perm.push_back(p.i64());
    Val o = make(dt, total);
    int rank = (int)shape.size();
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; ++i) {
      int64_t rem = i, aIdx = 0;
      for (int d = 0; d < rank; ++d) { int64_t c = rem / oStr[d]; rem -= c * oStr[d]; aIdx += c * aStr[perm[d]]; }
      o.raw[i] = a.raw[aIdx];
    }
    return o;
  }
  if (k == "matmul" || k == "matmul_batched") {
    const Val& a = V(op["a"].i32()); const Val& b = V(op["b"].i32());
    const Shape& as = SH(op["a"].i32()); const Shape& bs = SH(op["b"].i32());
    bool batched = k == "matmul_batched";
    int64_t M = as[as.size() - 2], K = as.back(), N = bs.back();
    int64_t batch = numel(as) / (M * K);
    Val o = make(F32, batch * M * N);
    const float* A = a.f(); const float* B = b.f();
    // Every output is s = ((0 + a0*b0) + a1*b1) + ... in increasing k, in f64 (the
    // evaluator's loop, _eval.ts:206-219); see matmul_f64.
    matmul_f64(A, B, o.f(), batch, M, K, N, batched);
    return o;
  }
  if (k == "one_hot") {
    const Val& idx = V(op["indices"].i32());
    int64_t D = op["depth"].i64();
    Val o = make(dt, total);
    for (size_t i = 0; i < idx.n(); ++i) { int64_t kk = idx.i()[i]; if (kk >= 0 && kk < D) store(o, i * D + kk, 1.0); }
    return o;
  }
  if (k == "less" || k == "greater") {
    const Val& a = V(op["a"].i32()); const Val& b = V(op["b"].i32());
    const Shape& as = SH(op["a"].i32()); const Shape& bs = SH(op["b"].i32());
    Val o = make(I32, total);
    bool lt = k == "less";
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; ++i) {
      double x = a.num(bidx(i, shape, as)), y = b.num(bidx(i, shape, bs));
      o.i()[i] = (lt ? x < y : x > y) ? 1 : 0;
    }
    return o;
  }
  if (k == "where") {
    const Val& c = V(op["cond"].i32()); const Val& a = V(op["a"].i32()); const Val& b = V(op["b"].i32());
    const Shape& cs = SH(op["cond"].i32()); const Shape& as = SH(op["a"].i32()); const Shape& bs = SH(op["b"].i32());
    Val o = make(dt, total);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; ++i) {
      int32_t cv = c.i()[bidx(i, shape, cs)];
      store(o, i, cv != 0 ? a.num(bidx(i, shape, as)) : b.num(bidx(i, shape, bs)));
    }
    return o;
  }
  if (k == "log_softmax_last") {
    const Val& a = V(op["a"].i32());
    const Shape& as = SH(op["a"].i32());
    int64_t D = as.back(), outer = numel(as) / D;
    Val o = make(F32, (int64_t)a.n());
    const float* A = a.f();
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < outer; ++i) {
      double mx = -INFINITY;
      for (int64_t j = 0; j < D; ++j) if ((double)A[i * D + j] > mx) mx = A[i * D + j];
      double se = 0;
      for (int64_t j = 0; j < D; ++j) se += std::exp((double)A[i * D + j] - mx);
      double ls = std::log(se) + mx;
      for (int64_t j = 0; j < D; ++j) o.f()[i * D + j] = (float)((double)A[i * D + j] - ls);
    }
    return o;
  }
  if (k == "softmax_causal_last") {
    const Val& a = V(op["a"].i32());
    const Shape& as = SH(op["a"].i32());
    int64_t D = as.back(), outer = numel(as) / (D * D);
    Val o = make(F32, (int64_t)a.n());
    const float* A = a.f();
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t bi = 0; bi < outer; ++bi)
      for (int64_t i = 0; i < D; ++i) {
        const float* row = A + bi * D * D + i * D;
        double mx = -INFINITY;
        for (int64_t j = 0; j <= i; ++j) if ((double)row[j] > mx) mx = row[j];
        double se = 0;
        for (int64_t j = 0; j <= i; ++j) se += std::exp((double)row[j] - mx);
        float* orow = o.f() + bi * D * D + i * D;
        for (int64_t j = 0; j < D; ++j) orow[j] = j <= i ? (float)(std::exp((double)row[j] - mx) / se) : 0.0f;
      }
    return o;
  }
  if (k == "where_causal") {
    const Val& a = V(op["a"].i32());
    const Shape& as = SH(op["a"].i32());
    int64_t D = as.back(), outer = numel(as) / (D * D);
    double fill = op["fillValue"].num();
    Val o = make(F32, (int64_t)a.n());
    for (int64_t bi = 0; bi < outer; ++bi)
      for (int64_t i = 0; i < D; ++i)
        for (int64_t j = 0; j < D; ++j) {
          int64_t q = bi * D * D + i * D + j;
          o.f()[q] = j <= i ? (float)a.num(q) : (float)fill;
        }
    return o;
  }
  if (k == "slice_range") {
    const Val& a = V(op["a"].i32());
    const Shape& as = SH(op["a"].i32());
    int64_t ax = op["axis"].i64(), st = op["start"].i64(), en = op["end"].i64();
    int64_t inner = 1; for (size_t d = ax + 1; d < as.size(); ++d) inner *= as[d];
    int64_t Din = as[ax], Dout = en - st, outer = numel(as) / (Din * inner);
    Val o = make(dt, outer * Dout * inner);
    for (int64_t i = 0; i < outer; ++i)
      for (int64_t j = 0; j < Dout; ++j)
        for (int64_t q = 0; q < inner; ++q) o.raw[(i * Dout + j) * inner + q] = a.raw[(i * Din + j + st) * inner + q];
    return o;
  }
  if (k == "scatter_axis") {
    const Val& a = V(op["a"].i32());
    int64_t ax = op["axis"].i64(), st = op["start"].i64(), en = op["end"].i64();
    int64_t inner = 1; for (size_t d = ax + 1; d < shape.size(); ++d) inner *= shape[d];
    int64_t Dout = shape[ax], Din = en - st, outer = total / (Dout * inner);
    Val o = make(dt, total);
    for (int64_t i = 0; i < outer; ++i)
      for (int64_t j = st; j < en; ++j)
        for (int64_t q = 0; q < inner; ++q) o.raw[(i * Dout + j) * inner + q] = a.raw[(i * Din + (j - st)) * inner + q];
    return o;
  }
  if (k == "concat") {
    int64_t ax = op["axis"].i64();
    int64_t inner = 1; for (size_t d = ax + 1; d < shape.size(); ++d) inner *= shape[d];
    int64_t Dout = shape[ax], outer = total / (Dout * inner);
    Val o = make(dt, total);
    int64_t off = 0;
    for (auto& idv : op["inputs"].a) {
      int id = idv.i32();
      const Val& a = V(id);
      int64_t Din = SH(id)[ax];
      for (int64_t i = 0; i < outer; ++i)
        for (int64_t j = 0; j < Din; ++j)
          for (int64_t q = 0; q < inner; ++q) o.raw[(i * Dout + off + j) * inner + q] = a.raw[(i * Din + j) * inner + q];
      off += Din;
    }
    return o;
  }
  if (k == "broadcast_to") {
    const Val& a = V(op["a"].i32());
    const Shape& as = SH(op["a"].i32());
    Val o = make(dt, total);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; ++i) o.raw[i] = a.raw[bidx(i, shape, as)];
    return o;
  }
  if (k == "sum_to_shape") {
    // f32 running sum in source-flat order (_eval.ts:492-523). Parallel over output cells:
    // each cell still visits its sources in increasing flat order.
    const Val& a = V(op["a"].i32());
    const Shape& as = SH(op["a"].i32());
    int64_t aTotal = numel(as);
    int64_t rankDiff = (int64_t)as.size() - (int64_t)shape.size();
    // Source dim d maps to output stride ostr[d] (0 where the output has size 1 or no
    // dim): the sources of a cell are a product set over the reduced dims, visited here
    // in increasing flat index (outer reduced dim slowest), as the evaluator's single
    // pass over the source does for each cell.
    const int64_t R = (int64_t)as.size();
    std::vector<int64_t> ostr(R, 0), astr(R, 1);
    {
      int64_t os = 1;
      for (int64_t d = (int64_t)shape.size() - 1; d >= 0; --d) {
        if (shape[d] != 1) ostr[d + rankDiff] = os;
        os *= shape[d];
      }
      for (int64_t d = R - 2; d >= 0; --d) astr[d] = astr[d + 1] * as[d + 1];
    }
    std::vector<int64_t> kept, reduced;   // source dims that index the output / that are summed
    for (int64_t d = 0; d < R; ++d) (ostr[d] ? kept : reduced).push_back(d);
    Val o = make(F32, total);
    if (aTotal == 0) return o;
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < total; ++c) {
      // decompose the cell over the kept dims (outer to inner)
      int64_t rem = c, base = 0;
      for (int64_t q = (int64_t)kept.size() - 1; q >= 0; --q) {
        const int64_t d = kept[q];
        const int64_t cd = rem % as[d];
        rem /= as[d];
        base += cd * astr[d];
      }
      float s = 0.0f;
      double sd = 0.0;   // the fixtures' f64-sum twin (orc_set_sum_f64): one rounding at the end
      std::vector<int64_t> ctr(reduced.size(), 0);
      for (;;) {
        int64_t off = base;
        for (size_t q = 0; q < reduced.size(); ++q) off += ctr[q] * astr[reduced[q]];
        if (g_sum_f64) sd += a.num(off);
        else s = (float)((double)s + a.num(off));
        int64_t q = (int64_t)reduced.size() - 1;
        for (; q >= 0; --q) {
          if (++ctr[q] < as[reduced[q]]) break;
          ctr[q] = 0;
        }
        if (q < 0) break;
      }
      o.f()[c] = g_sum_f64 ? (float)sd : s;
    }
    return o;
  }
  if (k == "relu_grad") {
    const Val& x = V(op["x"].i32()); const Val& dy = V(op["dy"].i32());
    Val o = make(F32, (int64_t)x.n());
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)x.n(); ++i) o.f()[i] = x.num(i) > 0 ? (float)dy.num(i) : 0.0f;
    return o;
  }
  if (k == "randn") {
    uint32_t seed = (uint32_t)V(op["seed"].i32()).i()[0];
    uint32_t sc = salt_const(op["salt"].i64());
    Val o = make(F32, total);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; ++i) {
      uint32_t h1, h2;
      pcg_imul2(seed, sc, (uint32_t)i, h1, h2);
      double u1 = std::max(1e-10, h1 / 4294967296.0), u2 = h2 / 4294967296.0;
      o.f()[i] = (float)(std::sqrt(-2 * std::log(u1)) * std::cos(2 * M_PI * u2));
    }
    return o;
  }
  if (k == "dropout") {
    const Val& a = V(op["a"].i32());
    uint32_t seed = (uint32_t)V(op["seed"].i32()).i()[0];
    uint32_t sc = salt_const(op["salt"].i64());
    double p = op["p"].num();
    double scale = 1 / (1 - p);
    Val o = make(F32, (int64_t)a.n());
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)a.n(); ++i) {
      uint32_t h = pcg_f64(seed, sc, (uint32_t)i);
      double u = h / 4294967296.0;
      double mask = u >= p ? scale : 0;
      o.f()[i] = (float)(a.num(i) * mask);
    }
    return o;
  }
  if (k == "categorical_last") {
    const Val& a = V(op["a"].i32());
    const Shape& as = SH(op["a"].i32());
    uint32_t seed = (uint32_t)V(op["seed"].i32()).i()[0];
    uint32_t sc = salt_const(op["salt"].i64());
    int64_t D = as.back(), outer = (int64_t)a.n() / D;
    Val o = make(I32, outer);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < outer; ++i) {
      double bv = -INFINITY; int64_t bi = 0;
      for (int64_t j = 0; j < D; ++j) {
        uint32_t h = pcg_f64(seed, sc, (uint32_t)(i * D + j));
        double u = std::max(1e-10, h / 4294967296.0);
        double g = -std::log(-std::log(u));
        double v = a.num(i * D + j) + g;
        if (v > bv) { bv = v; bi = j; }
      }
      o.i()[i] = (int32_t)bi;
    }
    return o;
  }
  if (k == "adam_update_m" || k == "adam_update_v") {
    bool isM = k == "adam_update_m";
    const Val& s = V(op[isM ? "m" : "v"].i32()); const Val& g = V(op["g"].i32());
    double beta = op[isM ? "beta1" : "beta2"].num(), omb = 1 - beta;
    Val o = make(F32, total);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; ++i) {
      double gv = g.f()[i];
      double r = isM ? beta * (double)s.f()[i] + omb * gv : beta * (double)s.f()[i] + omb * gv * gv;
      o.f()[i] = (float)r;
    }
    return o;
  }
  if (k == "adam_update_p") {
    const Val& p = V(op["p"].i32()); const Val& m = V(op["mNew"].i32()); const Val& v = V(op["vNew"].i32());
    double lrt = V(op["lrt"].i32()).f()[0];
    double eps = op["eps"].num();
    const JV& dst = op["decayShrinkTensor"];
    double shrink = dst.is_null() ? op["decayShrink"].num() : (double)V(dst.i32()).f()[0];
    Val o = make(F32, total);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; ++i) {
      double r = shrink * (double)p.f()[i] - lrt * (double)m.f()[i] / (std::sqrt((double)v.f()[i]) + eps);
      o.f()[i] = (float)r;
    }
    return o;
  }
  if (k == "conv2d") {
    int inId = op["input"].i32(), wId = op["weight"].i32();
    const float* X = V(inId).f(); const float* Wt = V(wId).f();
    const Shape& is = SH(inId); const Shape& ws = SH(wId);
    int64_t cIn = is[1], H = is[2], W = is[3], cOut = ws[0], cInPG = ws[1], kH = ws[2], kW = ws[3];
    int64_t G = op["groups"].i64(), cOutPG = cOut / G;
    int64_t sH = op["strideH"].i64(), sW = op["strideW"].i64(), pH = op["padH"].i64(), pW = op["padW"].i64();
    int64_t B = shape[0], hO = shape[2], wO = shape[3];
    Val o = make(F32, total);
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < B; ++b)
      for (int64_t co = 0; co < cOut; ++co)
        for (int64_t ho = 0; ho < hO; ++ho)
          for (int64_t wo = 0; wo < wO; ++wo) {
            int64_t g = co / cOutPG;
            double s = 0;
            for (int64_t cl = 0; cl < cInPG; ++cl)
              for (int64_t kh = 0; kh < kH; ++kh) {
                int64_t ci = g * cInPG + cl, hi = ho * sH + kh - pH;
                if (hi < 0 || hi >= H) continue;
                for (int64_t kw = 0; kw < kW; ++kw) {
                  int64_t wi = wo * sW + kw - pW;
                  if (wi < 0 || wi >= W) continue;
                  s += (double)X[((b * cIn + ci) * H + hi) * W + wi] * (double)Wt[((co * cInPG + cl) * kH + kh) * kW + kw];
                }
              }
            o.f()[((b * cOut + co) * hO + ho) * wO + wo] = (float)s;
          }
    return o;
  }
  if (k == "conv2d_input_grad") {
    int wId = op["weight"].i32(), dyId = op["dy"].i32();
    const float* Wt = V(wId).f(); const float* DY = V(dyId).f();
    const Shape& ws = SH(wId); const Shape& dys = SH(dyId);
    int64_t cOut = ws[0], cInPG = ws[1], kH = ws[2], kW = ws[3];
    int64_t G = op["groups"].i64(), cOutPG = cOut / G;
    int64_t sH = op["strideH"].i64(), sW = op["strideW"].i64(), pH = op["padH"].i64(), pW = op["padW"].i64();
    int64_t hO = dys[2], wO = dys[3];
    int64_t B = shape[0], cIn = shape[1], inH = shape[2], inW = shape[3];
    Val o = make(F32, total);
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < B; ++b)
      for (int64_t ci = 0; ci < cIn; ++ci)
        for (int64_t hi = 0; hi < inH; ++hi)
          for (int64_t wi = 0; wi < inW; ++wi) {
            int64_t g = ci / cInPG, cl = ci - g * cInPG;
            double s = 0;
            for (int64_t col = 0; col < cOutPG; ++col) {
              int64_t co = g * cOutPG + col;
              for (int64_t kh = 0; kh < kH; ++kh) {
                int64_t nh = hi + pH - kh;
                if (nh < 0 || nh % sH != 0) continue;
                int64_t ho = nh / sH;
                if (ho >= hO) continue;
                for (int64_t kw = 0; kw < kW; ++kw) {
                  int64_t nw = wi + pW - kw;
                  if (nw < 0 || nw % sW != 0) continue;
                  int64_t wo = nw / sW;
                  if (wo >= wO) continue;
                  s += (double)Wt[((co * cInPG + cl) * kH + kh) * kW + kw] * (double)DY[((b * cOut + co) * hO + ho) * wO + wo];
                }
              }
            }
            o.f()[((b * cIn + ci) * inH + hi) * inW + wi] = (float)s;
          }
    return o;
  }
  if (k == "conv2d_weight_grad") {
    int inId = op["input"].i32(), dyId = op["dy"].i32();
    const float* X = V(inId).f(); const float* DY = V(dyId).f();
    const Shape& is = SH(inId); const Shape& dys = SH(dyId);
    int64_t B = is[0], cIn = is[1], H = is[2], W = is[3], cOut = dys[1], hO = dys[2], wO = dys[3];
    int64_t cInPG = shape[1], kH = shape[2], kW = shape[3];
    int64_t G = op["groups"].i64(), cOutPG = cOut / G;
    int64_t sH = op["strideH"].i64(), sW = op["strideW"].i64(), pH = op["padH"].i64(), pW = op["padW"].i64();
    Val o = make(F32, total);
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t co = 0; co < cOut; ++co)
      for (int64_t cl = 0; cl < cInPG; ++cl)
        for (int64_t kh = 0; kh < kH; ++kh)
          for (int64_t kw = 0; kw < kW; ++kw) {
            int64_t g = co / cOutPG, ci = g * cInPG + cl;
            double s = 0;
            for (int64_t b = 0; b < B; ++b)
              for (int64_t ho = 0; ho < hO; ++ho) {
                int64_t hi = ho * sH + kh - pH;
                if (hi < 0 || hi >= H) continue;
                for (int64_t wo = 0; wo < wO; ++wo) {
                  int64_t wi = wo * sW + kw - pW;
                  if (wi < 0 || wi >= W) continue;
                  s += (double)X[((b * cIn + ci) * H + hi) * W + wi] * (double)DY[((b * cOut + co) * hO + ho) * wO + wo];
                }
              }
            o.f()[((co * cInPG + cl) * kH + kh) * kW + kw] = (float)s;
          }
    return o;
  }
  if (k == "max_pool_2d") {
    int inId = op["input"].i32();
    const float* X = V(inId).f();
    const Shape& is = SH(inId);
    int64_t B = is[0], C = is[1], H = is[2], W = is[3], hO = shape[2], wO = shape[3];
    int64_t kH = op["kH"].i64(), kW = op["kW"].i64(), sH = op["strideH"].i64(), sW = op["strideW"].i64();
    int64_t pH = op["padH"].i64(), pW = op["padW"].i64();
    Val o = make(F32, total);
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < B; ++b)
      for (int64_t c = 0; c < C; ++c)
        for (int64_t ho = 0; ho < hO; ++ho)
          for (int64_t wo = 0; wo < wO; ++wo) {
            double m = -3.4e38;
            for (int64_t kh = 0; kh < kH; ++kh) {
              int64_t hi = ho * sH + kh - pH;
              if (hi < 0 || hi >= H) continue;
              for (int64_t kw = 0; kw < kW; ++kw) {
                int64_t wi = wo * sW + kw - pW;
                if (wi < 0 || wi >= W) continue;
                double v = X[((b * C + c) * H + hi) * W + wi];
                if (v > m) m = v;
              }
            }
            o.f()[((b * C + c) * hO + ho) * wO + wo] = (float)m;
          }
    return o;
  }
  if (k == "max_pool_2d_grad") {
    int inId = op["input"].i32(), dyId = op["dy"].i32();
    const float* X = V(inId).f(); const float* DY = V(dyId).f();
    const Shape& is = SH(inId); const Shape& dys = SH(dyId);
    int64_t B = is[0], C = is[1], H = is[2], W = is[3], hO = dys[2], wO = dys[3];
    int64_t kH = op["kH"].i64(), kW = op["kW"].i64(), sH = op["strideH"].i64(), sW = op["strideW"].i64();
    int64_t pH = op["padH"].i64(), pW = op["padW"].i64();
    Val o = make(F32, total);
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < B; ++b)
      for (int64_t c = 0; c < C; ++c)
        for (int64_t hi = 0; hi < H; ++hi)
          for (int64_t wi = 0; wi < W; ++wi) {
            double s = 0;
            for (int64_t kh = 0; kh < kH; ++kh) {
              int64_t nh = hi + pH - kh;
              if (nh < 0 || nh % sH != 0) continue;
              int64_t ho = nh / sH;
              if (ho >= hO) continue;
              for (int64_t kw = 0; kw < kW; ++kw) {
                int64_t nw = wi + pW - kw;
                if (nw < 0 || nw % sW != 0) continue;
                int64_t wo = nw / sW;
                if (wo >= wO) continue;
                double m = -3.4e38; int64_t ah = -1, aw = -1;
                for (int64_t kkh = 0; kkh < kH; ++kkh) {
                  int64_t hh = ho * sH + kkh - pH;
                  if (hh < 0 || hh >= H) continue;
                  for (int64_t kkw = 0; kkw < kW; ++kkw) {
                    int64_t ww = wo * sW + kkw - pW;
                    if (ww < 0 || ww >= W) continue;
                    double v = X[((b * C + c) * H + hh) * W + ww];
                    if (v > m) { m = v; ah = hh; aw = ww; }
                  }
                }
                if (ah == hi && aw == wi) s += (double)DY[((b * C + c) * hO + ho) * wO + wo];
              }
            }
            o.f()[((b * C + c) * H + hi) * W + wi] = (float)s;
          }
    return o;
  }
  throw std::runtime_error("eval: unhandled op kind " + k);
}

}  // namespace orc

// ---- C ABI for ctypes (tests, smoke, bench cpu_baseline) --------------------------------

using orc::Oracle;
using orc::Val;

extern "C" {

const char* orc_last_error() { return orc::g_err.c_str(); }

void orc_set_matmul_f32(int on) { orc::g_matmul_f32 = on != 0; }
void orc_set_sum_f64(int on) { orc::g_sum_f64 = on != 0; }

void orc_set_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n > 0 ? n : 1);
#else
  (void)n;
#endif
}

int orc_max_threads() {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void* orc_create(const char* wire_json) {
  try { return new Oracle(wire_json); } catch (std::exception& e) { orc::g_err = e.what(); return nullptr; }
}

void orc_destroy(void* h) { delete static_cast<Oracle*>(h); }

int orc_num_params(void* h) { return (int)static_cast<Oracle*>(h)->params().size(); }
const char* orc_param_name(void* h, int i) { return static_cast<Oracle*>(h)->params().at(i).c_str(); }

// Param or optimizer-state home buffer access (f32).
int orc_set_home(void* h, const char* name, const float* data, int64_t n) {
  try {
    Val& v = static_cast<Oracle*>(h)->home(name);
    if ((int64_t)v.n() != n) { orc::g_err = std::string("size mismatch for ") + name; return -1; }
    memcpy(v.raw.data(), data, n * 4);
    return 0;
  } catch (std::exception& e) { orc::g_err = e.what(); return -1; }
}

int orc_get_home(void* h, const char* name, float* out, int64_t n) {
  try {
    Val& v = static_cast<Oracle*>(h)->home(name);
    if ((int64_t)v.n() != n) { orc::g_err = std::string("size mismatch for ") + name; return -1; }
    memcpy(out, v.raw.data(), n * 4);
    return 0;
  } catch (std::exception& e) { orc::g_err = e.what(); return -1; }
}

static std::map<std::string, Val> make_inputs(int n, const char** names, const void** data, const int64_t* nbytes) {
  std::map<std::string, Val> m;
  for (int i = 0; i < n; ++i) {
    Val v; v.dt = orc::F32;
    v.raw.resize(nbytes[i] / 4);
    memcpy(v.raw.data(), data[i], nbytes[i]);
    m[names[i]] = v;
  }
  return m;
}

int orc_step(void* h, int n, const char** names, const void** data, const int64_t* nbytes, double* loss) {
  try {
    *loss = static_cast<Oracle*>(h)->step(make_inputs(n, names, data, nbytes));
    return 0;
  } catch (std::exception& e) { orc::g_err = e.what(); return -1; }
}

int orc_run(void* h, int n, const char** names, const void** data, const int64_t* nbytes) {
  try {
    static_cast<Oracle*>(h)->run(make_inputs(n, names, data, nbytes));
    return 0;
  } catch (std::exception& e) { orc::g_err = e.what(); return -1; }
}

void orc_retain_all(void* h, int on) { static_cast<Oracle*>(h)->retain_all(on != 0); }
int orc_output_tid(void* h) { return static_cast<Oracle*>(h)->output_tid(); }

// Copy tensor `tid` from the last evaluation (4-byte elements).
int orc_get_tensor(void* h, int tid, void* out, int64_t nbytes) {
  try {
    const Val& v = static_cast<Oracle*>(h)->value(tid);
    if ((int64_t)v.n() * 4 != nbytes) { orc::g_err = "size mismatch"; return -1; }
    memcpy(out, v.raw.data(), nbytes);
    return 0;
  } catch (std::exception& e) { orc::g_err = e.what(); return -1; }
}

int orc_set_lr(void* h, const char* lr_json) {
  try { static_cast<Oracle*>(h)->set_lr(lr_json); return 0; } catch (std::exception& e) { orc::g_err = e.what(); return -1; }
}

void orc_reset_optimizer(void* h) { static_cast<Oracle*>(h)->reset_optimizer(); }

// PRNG primitives, exposed for known-answer tests.
uint32_t orc_pcg_f64(uint32_t seed, uint32_t salt_const, uint32_t idx) { return orc::pcg_f64(seed, salt_const, idx); }
void orc_pcg_imul2(uint32_t seed, uint32_t salt_const, uint32_t idx, uint32_t* h1, uint32_t* h2) {
  orc::pcg_imul2(seed, salt_const, idx, *h1, *h2);
}
uint32_t orc_salt_const(int64_t salt) { return orc::salt_const(salt); }
double orc_resolve_lr(const char* lr_json, double step) {
  try { return orc::resolve_lr(orc::parse_json(lr_json), step); } catch (std::exception& e) { orc::g_err = e.what(); return NAN; }
}

}  // extern "C"
