// Host runtime of the gfx950 backend: reads the traced IR, plans device memory, lowers
// IR ops to HIP kernel launches, captures the whole step as one hipGraph and serves the
// C ABI in include/tg.h.
//
// It takes the place of the reference's buffer planner (src/buffers.ts), WGSL codegen
// (src/codegen.ts), WebGPU runtime (src/runtime.ts) and worker request handlers
// (src/worker.ts). Design, MI355X-first rather than one dispatch per IR op:
//  * views: reshape / stop_gradient / identity sum_to_shape and broadcast_to alias their
//    input; permute is a strided view that GEMMs and element-wise kernels read in place
//    and is materialised only for consumers that need contiguous rows;
//  * patterns: one_hot -> matmul becomes a row gather (embedding forward) and
//    transpose(one_hot) -> matmul a segmented scatter-add (embedding gradient), so the
//    one-hot matrix is never built for them; all adam_update_{m,v,p} ops become one fused
//    multi-tensor kernel updating p, m and v in place (no writeback copies);
//  * fusion: maximal convex runs of same-shape pointwise ops become one launch of the
//    fused register-machine kernel (k_fused.hip), storing only values used outside;
//  * memory: one arena per runtime, persistent regions for params / optimizer state /
//    inputs, and liveness-pooled intermediates (best fit, as buffers.ts:151-209);
//  * execution: one HIP stream; the launch sequence is captured once into a hipGraph
//    and replayed per step; per-step host work is one H2D copy of the input region
//    (user inputs + lrt / decayShrink / lr / PRNG seed scalars) and a 4-byte loss read.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/tg.h"
#include "json.hpp"
#include "jit.h"
#include "kernels.h"
#include "safetensors.hpp"

// Device scratch of the scratch-only step (tg_step_noalloc): split-K partials, reduction
// partials, the embedding-gradient sort and the launch-completion counters of one step
// live here instead of in memory the runtime allocates. One copy per GPU, held until the
// process ends. Host code never passes the array's name to a kernel (on the host it is a
// stand-in, not a device address): it uses the address hipGetSymbolAddress returns for
// the current device (scratch_address).
static constexpr size_t tg_kScratchBytes = (size_t)TG_SCRATCH_BYTES;

tgk::LaunchTimer*& tgk::launch_timer() {
  static thread_local LaunchTimer* t = nullptr;
  return t;
}
static __device__ __align__(256) unsigned char scratch[tg_kScratchBytes];

namespace tg {

static thread_local std::string g_error;

// Per-device address of `scratch`, looked up once per device with that device current.
static char* scratch_address() {
  static std::mutex mu;
  static std::map<int, char*> addr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) throw std::runtime_error(std::string("hipGetDevice: ") + hipGetErrorString(e));
  std::lock_guard<std::mutex> g(mu);
  auto it = addr.find(dev);
  if (it != addr.end()) return it->second;
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) throw std::runtime_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
  addr[dev] = static_cast<char*>(p);
  return static_cast<char*>(p);
}

// Scratch-only calls share the one array per GPU; calls from this process are serialised.
static std::mutex g_noalloc_mu;

struct Error : std::runtime_error {
  tg_status code;
  Error(tg_status c, const std::string& m) : std::runtime_error(m), code(c) {}
};

static void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Error(TG_DEVICE_ERROR, std::string(what) + ": " + hipGetErrorString(e));
}

enum Dt { F32 = 0, I32 = 1, BOOL = 2 };
static Dt parse_dt(const std::string& s) {
  if (s == "f32") return F32;
  if (s == "i32") return I32;
  if (s == "bool") return BOOL;
  throw Error(TG_INVALID_ARGUMENT, "IR: unknown dtype '" + s + "'");
}
static int kdt(Dt d) { return d == F32 ? tgk::DT_F32 : tgk::DT_I32; }

using Dims = std::vector<int64_t>;
static int64_t prod(const Dims& d) { int64_t n = 1; for (auto x : d) n *= x; return n; }
static Dims contiguous_strides(const Dims& d) {
  Dims s(d.size(), 1);
  for (int i = (int)d.size() - 2; i >= 0; --i) s[i] = s[i + 1] * d[i + 1];
  return s;
}

// Host-side bounds proof for every launch: the largest element offset an operand
// descriptor can produce must lie inside its root allocation.
static void check_span(const char* what, int64_t root_numel, int64_t base, const int64_t* dims, const int64_t* strides,
                       int rank) {
  int64_t hi = base, lo = base;
  for (int d = 0; d < rank; ++d) {
    if (dims[d] <= 0) return;   // empty iteration space touches nothing
    int64_t ext = (dims[d] - 1) * strides[d];
    if (ext >= 0) hi += ext; else lo += ext;
  }
  if (lo < 0 || hi >= std::max<int64_t>(root_numel, 1))
    throw Error(TG_INTERNAL, std::string("bounds check failed for ") + what + ": offsets [" + std::to_string(lo) + ", " +
                                 std::to_string(hi) + "] outside [0, " + std::to_string(root_numel) + ")");
}

// ---- learning-rate schedules (src/lr.ts:69-112) ---------------------------------------
static double resolve_lr(const tgj::Value& s, double step) {
  if (s.kind == tgj::Value::Number) return s.number;
  const std::string& k = s.at("kind").str();
  const tgj::Value* ss = s.get("startStep");
  double start = (ss && !ss->null()) ? ss->num() : 0;
  double st = std::max(1.0, step - start);
  if (k == "linear") {
    double f = std::min(st / s.at("steps").num(), 1.0);
    return s.at("peak").num() + (s.at("final").num() - s.at("peak").num()) * f;
  }
  if (k == "cosineAnnealing") {
    double f = std::min(st / s.at("steps").num(), 1.0);
    return s.at("final").num() + 0.5 * (s.at("peak").num() - s.at("final").num()) * (1 + std::cos(M_PI * f));
  }
  if (k == "warmup") {
    if (st <= s.at("steps").num()) return s.at("peak").num() * (st / s.at("steps").num());
    return resolve_lr(s.at("after"), st - s.at("steps").num());
  }
  if (k == "staircase") {
    double kk = std::floor((st - 1) / s.at("every").num());
    return s.at("peak").num() * std::pow(s.at("gamma").num(), kk);
  }
  if (k == "multiStep") {
    double kk = 0;
    for (const auto& m : s.at("milestones").items) if (st >= m.num()) kk += 1;
    return s.at("peak").num() * std::pow(s.at("gamma").num(), kk);
  }
  throw Error(TG_INVALID_ARGUMENT, "lr: unknown schedule kind '" + k + "'");
}

// Rebase a schedule so its intrinsic step 1 is `base` (src/lr.ts:108-112).
static tgj::Value rebase_lr(tgj::Value s, long long base) {
  if (s.kind == tgj::Value::Number) return s;
  const tgj::Value* ss = s.get("startStep");
  if (ss && !ss->null()) return s;
  tgj::Value v;
  v.kind = tgj::Value::Number;
  v.number = (double)(base - 1);
  bool set = false;
  for (auto& m : s.members) if (m.first == "startStep") { m.second = v; set = true; }
  if (!set) s.members.emplace_back("startStep", v);
  return s;
}

// ---- IR ----------------------------------------------------------------------------------
struct TInfo {
  Dims shape;
  Dt dt;
  int64_t numel;
  int src;  // producing op index
};

// A tensor as a strided view of a root tensor's storage (element strides, 4-byte elems).
struct View {
  int root;
  Dims dims, strides;
  bool contiguous() const {
    Dims c = contiguous_strides(dims);
    for (size_t i = 0; i < dims.size(); ++i) if (dims[i] != 1 && strides[i] != c[i]) return false;
    return true;
  }
};

struct Node {
  std::string kind;   // kernel family, for profiling / description
  int op = -1;        // IR op index it came from (the last one for fused nodes)
  std::vector<int> reads, writes;   // storage roots
  double flops = 0, bytes = 0;      // algorithmic work per launch
  std::string shape;
  std::string detail;  // fused groups: member op kinds in program order
  bool ws = false;     // bind() reads cur_ws_ / cur_counters_ (rebound for the scratch-only step)
  std::function<void(hipStream_t)> launch;   // bound after allocation
  std::function<std::function<void(hipStream_t)>()> bind;
};

class Runtime;

class Runtime {
 public:
  Runtime(const char* json, Runtime* parent, bool plan_only = false);
  ~Runtime();

  // parameters
  std::vector<std::string> param_names;
  std::map<std::string, int> param_root;      // name -> tensor id of the param_input
  int64_t param_numel(int i) const { return T_[param_root.at(param_names[i])].numel; }

  void upload_params(int n, const char* const* names, const float* const* data, const int64_t* numel);
  void download_params(int n, const char* const* names, float* const* data, const int64_t* numel);
  float step(int n, const char* const* names, const void* const* data, const int64_t* nbytes, bool device);
  float step_noalloc(int n, const char* const* names, const void* const* data, const int64_t* nbytes);
  void run(int n, const char* const* names, const void* const* data, const int64_t* nbytes, void* out, int64_t out_bytes);
  void get_capture(const std::string& name, void* out, int64_t nbytes);
  void reset_optimizer();
  void set_lr(const char* json);

  // Optimizer state (state_input tensors: Adam m / v, SGD velocity) in name order, plus
  // the step counter t and the PRNG seed counter, for checkpoints.
  const std::vector<std::string>& state_names() const;
  int64_t state_numel(const std::string& name) const;
  void download_state(int n, const char* const* names, float* const* data, const int64_t* numel);
  void upload_state(int n, const char* const* names, const float* const* data, const int64_t* numel);
  long long step_count() const { return t_; }
  long long prng_count() const { return prng_counter_; }
  void set_counters(long long t, long long prng) { t_ = t; prng_counter_ = prng; }
  void save_checkpoint(const std::string& path);
  void load_checkpoint(const std::string& path);
  std::string check_checkpoint_file(const std::string& path) const;
  std::string describe();
  void profile_nodes(int iters, double* ms, int64_t n);
  void profile_kernels(int iters, double* ms, int64_t n);
  double time_replays(int steps);
  double time_kinds(const std::string& kinds, int iters, int* launches);

  std::vector<std::string> capture_names;
  std::vector<Runtime*> children;
  Runtime* parent = nullptr;
  bool destroyed = false;

 private:
  tgj::Value doc_;
  std::vector<TInfo> T_;
  std::vector<const tgj::Value*> ops_;
  std::vector<std::string> kinds_;
  std::vector<std::vector<int>> consumers_;
  std::vector<View> view_;           // per tensor
  std::vector<bool> virtual_;        // op not executed (view / folded pattern)
  std::vector<bool> materialize_;    // permute output that needs its own storage
  std::map<std::string, int> input_tid_, state_tid_;
  std::vector<std::string> state_list_;   // state_tid_'s names, for the C ABI
  std::vector<int> outputs_;
  std::map<std::string, int> captures_;
  std::vector<std::pair<int, std::string>> copy_writebacks_;  // (source tid, dest name) applied by copy
  std::vector<Node> nodes_;

  // optimizer
  std::string opt_kind_;
  const tgj::Value* opt_cfg_ = nullptr;
  tgj::Value lr_;
  long long t_ = 0;
  bool uses_prng_ = false;
  long long prng_counter_ = 0;

  // device memory
  hipStream_t stream_ = nullptr;
  char* arena_ = nullptr;
  size_t arena_bytes_ = 0;
  std::vector<void*> ptr_;          // per root tensor
  char* input_region_ = nullptr;    // device: user inputs, then per-step scalars
  size_t input_region_bytes_ = 0;
  size_t user_bytes_ = 0;           // user inputs occupy [0, user_bytes_)
  std::vector<char*> slots_;        // device-resident staged batches (user part only)
  std::map<int, size_t> input_offset_;   // input tid -> byte offset in region
  char* staging_ = nullptr;         // pinned host mirror of the input region
  float* loss_host_ = nullptr;      // pinned
  float* workspace_ = nullptr;
  size_t workspace_bytes_ = 0;
  // Launch-completion counters (zeroed once; every kernel that counts on them leaves them
  // zero). Nodes reserve slots while lowering.
  int64_t counter_slots_ = 0;
  unsigned* counters_ = nullptr;
  int64_t take_counters(int64_t n) {
    const int64_t b = counter_slots_;
    counter_slots_ += n;
    return b;
  }
  // Column partial sums written by GEMM epilogues and read by the deferred column-sum
  // launch of the same step: a region of its own, allocated once (byte offsets, 256-byte
  // aligned), never pooled.
  size_t partial_bytes_ = 0;
  char* partials_ = nullptr;
  size_t take_partials(size_t bytes) {
    const size_t b = partial_bytes_;
    partial_bytes_ += (bytes + 255) & ~(size_t)255;
    return b;
  }
  struct CkptPlan {
    tgst::Index ix;
    std::vector<std::pair<size_t, int>> writes;   // (index in ix.tensors, tensor id)
    size_t n_state = 0;
    long long t = 0, c = 0;
    tgj::Value lr;
  };
  CkptPlan check_checkpoint(const std::vector<uint8_t>& buf) const;
  std::map<std::string, std::pair<void*, size_t>> table_cache_;   // dev_table copies by key
  const void* dev_table(const std::string& key, const void* data, size_t bytes);
  std::vector<int> state_roots_;

  hipGraph_t graph_ = nullptr;
  hipGraphExec_t graph_exec_ = nullptr;
  bool plan_only_ = false;

  // Element-wise fusion groups: members in op order; the group runs at its first op.
  // A fused group: ops evaluated by one launch of the fused kernel. `shape` is the
  // iteration shape: every member's output for an element group; for a row group (one
  // that contains last-axis reductions) the full [.., D] shape, members producing either
  // that shape or its row shape ([..] or [.., 1]).
  // `dups` are pointwise ops of other groups that this element group evaluates again from
  // their inputs instead of reading their results (never stored here).
  struct Group { int first; std::vector<int> ops; Dims shape; bool row = false; std::vector<int> dups; };
  // Register plan of a group: external operands (tensor + the broadcast class of the
  // consumer: 0 full, 1 row [..], 2 row [.., 1]), stored outputs, and a linear-scan
  // register assignment (a register is reused after its value's last read).
  struct GroupPlan {
    std::vector<std::pair<int, int>> ext;   // (tensor, class) loaded into registers 0..n-1
    int seed = -1;
    std::vector<int> outs;                  // member outputs stored by the launch
    std::vector<int> out_reg;
    std::vector<tgk::FusedInstr> code;
    int nregs = 0;
  };
  GroupPlan plan_group(const std::vector<int>& ops, bool row, const Dims& F,
                       const std::vector<int>* dups = nullptr) const;
  bool dup_in(int gi, int m) const;
  std::vector<char> dropped_;   // op left out of its own group: only groups recomputing it run it
  int producer_group(int t) const;
  int op_class(int m, bool row, const Dims& F) const;
  int inline_one_hot(int t, const Dims& F) const;
  bool is_row_reduce(int m) const;
  std::vector<Group> groups_;
  std::vector<int> group_of_;   // op -> group index or -1
  // Fused attention: matmul_batched(q, k^T) [-> mul_scalar] -> softmax_causal_last
  // [-> dropout] -> matmul_batched(., v), run as one node at the first product.
  struct AttnMatch { int qk, scale, softmax, dropout, pv; };
  std::vector<AttnMatch> attn_;
  std::vector<int> attn_of_;    // op -> attention match or -1 (forward and backward chains)
  void match_attention();
  void lower_attention(int m);
  // The backward of a matched chain: dPd = dO V^T, dropout, softmax backward row ops,
  // dQ = dS K, dK^T = Q^T dS, dV = Pd^T dO, run as one node at its first op.
  struct AttnBwd { int fwd, first, dpd, dq, dkt, dv, ds_op; std::vector<int> ops; };
  std::vector<AttnBwd> attn_bwd_;
  void match_attention_bwd();
  void lower_attention_bwd(int m);
  // Column sums (sum_to_shape over a leading block of dims of a contiguous tensor): a
  // single-use f32 product feeding one is absorbed (the kernel multiplies), and sums of
  // the same shape whose inputs are ready are launched together.
  struct ColSumOp { int a, b; int64_t R, C; };   // b >= 0: sum of the product a * b
  std::map<int, ColSumOp> colsum_;
  // Deferred column sums whose operand is an output of a GEMM epilogue: that epilogue writes
  // f64 column partials (`rows` rows at byte offset `off` of partials_), which the
  // column-sum launch adds instead of reading the operand back.
  struct ColPart { size_t off; int64_t rows; };
  std::map<int, ColPart> colsum_part_;
  bool use_colsum_epi_ = true;       // TG_COLSUM_EPI=0: the column sums read their operands
  std::vector<bool> colsum_done_, mul_absorbed_;
  void match_colsums();
  // Sums of products: an add tree ((p1 + p2) + p3 ..) over single-use GEMM products of one
  // shape runs as one GEMM over the products' concatenated k ranges (gemm_sum), emitted at
  // the final add; the products and the inner adds are absorbed.
  bool use_gemm_sum_ = true;         // TG_GEMM_SUM=0 keeps the products and adds apart
  std::map<int, std::vector<int>> gemm_sums_;   // final add -> matmul ops, in k order
  // Products reading a last-axis concatenation [R, k0 + k1] of two sources as their A
  // operand: run as one GEMM over the sources (tgk::gemm_cat). A concatenation all of whose
  // readers are such products or per-source weight gradients is not materialised.
  struct CatFwd { int src0, src1; int64_t k0, k1; };
  std::map<int, CatFwd> cat_fwd_;     // matmul op -> its A's sources
  std::vector<char> cat_absorbed_;    // concat op -> not lowered
  std::vector<char> pool_absorbed_;   // relu_grad op applied by the max-pool gradient launch before it
  void match_concat_products();
  void check_cat_spans(const tgk::GemmDesc& d, const CatFwd& c, int b, int out, bool with_c) const;
  std::vector<char> sum_absorbed_;
  void match_gemm_sums();
  void lower_gemm_sum(int add_op);
  void lower_colsums(int s);
  int emit_pos(int op) const;
  std::deque<tgk::FusedProgram> programs_;     // kernel-argument images (stable addresses)
  std::vector<tgk::FusedInstr> fused_code_;    // all groups' instructions, uploaded once
  tgk::FusedInstr* fused_code_dev_ = nullptr;
  // Fused groups run as kernels generated per group (default) or, with TG_FUSED=vm in
  // the environment, through the interpreter kernels of k_fused.hip.
  bool use_jit_ = true;
  bool use_conv_gemm_ = true;   // implicit-GEMM convolutions (TG_CONV=direct: direct f64 kernels)
  struct JitSlot {
    std::string name;
    hipFunction_t fn = nullptr;
    tgk::JitArgs args{};
    int64_t grid = 0;
    bool gemm = false;          // a GEMM with a fused epilogue: launched with gargs first
    int threads = 256;
    tgk::gd::GemmArgs gargs{};
  };
  std::deque<JitSlot> jit_slots_;
  std::vector<tgk::JitKernel> jit_pending_;
  void jit_finish();
  void launch_jit(size_t js, hipStream_t st) {
    JitSlot& j = jit_slots_[js];
    void* p1[] = {&j.args};
    void* p2[] = {&j.gargs, &j.args};
    hipEvent_t a = nullptr, b = nullptr;
    tgk::LaunchTimer* t = tgk::launch_timer();
    // hipExtModuleLaunchKernel takes the global work size (blocks x threads per block)
    const hipError_t e =
        t && t->take(a, b)
            ? hipExtModuleLaunchKernel(j.fn, (uint32_t)(j.grid * j.threads), 1, 1, (uint32_t)j.threads, 1, 1, 0, st,
                                       j.gemm ? p2 : p1, nullptr, a, b, 0)
            : hipModuleLaunchKernel(j.fn, (unsigned)j.grid, 1, 1, (unsigned)j.threads, 1, 1, 0, st, j.gemm ? p2 : p1,
                                    nullptr);
    if (e != hipSuccess) throw Error(TG_DEVICE_ERROR, std::string("generated kernel launch: ") + hipGetErrorString(e));
  }
  void form_groups();
  void merge_groups();
  void remat_groups();
  void lower_group(int gi);

  bool is_leaf(int op) const {
    const std::string& k = kinds_[op];
    return k == "param_input" || k == "tensor_input" || k == "state_input";
  }
  // Tensors that depend on constants only (no input, parameter, state or random op): their
  // producers can be lowered ahead of their positions (the nodes then run once, among the
  // init nodes). const_early_ok: every producer of t not lowered yet is such an op, on its
  // own or in a group of such ops only; lower_const_early lowers them, inputs first.
  bool const_early_ok(int t, int depth = 0) const;
  void lower_const_early(int t);
  int root(int t) const { return view_[t].root; }
  void* dptr(int t) const { return ptr_[root(t)]; }
  const tgj::Value& O(int op) const { return *ops_[op]; }
  int fld(int op, const char* f) const { return O(op).at(f).i32(); }

  void read_document();
  void analyse();
  void relu_grads_from_outputs();
  void narrow_sliced_products();
  bool concat_transposed(int t, std::vector<int>& srcs, std::vector<int64_t>& offs) const;
  void compute_views();
  void lower();
  void allocate();
  void bind_all();
  // Launches whose results do not change between steps (constants and what is computed
  // only from them, e.g. the loss gradient seed) run once after the buffers are bound;
  // their outputs live in the persistent region.
  std::vector<Node> init_nodes_;
  std::set<int> init_roots_;
  void split_init_nodes();
  void launch_all(hipStream_t st);
  void upload_inputs(int n, const char* const* names, const void* const* data, const int64_t* nbytes, bool device);
  void advance_scalars(bool optimizer);
  void upload_scalars();
 public:
  void stage_batch(int slot, int n, const char* const* names, const void* const* data, const int64_t* nbytes);
  float step_staged(int slot);
 private:
  void ensure_graph();
  void replay();
  float* cur_ws_ = nullptr;            // workspace of the node being bound
  unsigned* cur_counters_ = nullptr;   // launch-completion counters of the node being bound
  // Scratch-only step (tg_step_noalloc): the launches again, with every node that uses the
  // workspace or the counters bound to the library's static device scratch instead.
  std::vector<std::function<void(hipStream_t)>> noalloc_launch_;
  std::string noalloc_error_;
  unsigned* noalloc_counters_ = nullptr;
  void prepare_noalloc();
  // TG_GRAPH=0 in the environment issues each step's launches directly instead of
  // replaying a captured hipGraph (for tools that do not follow graph launches).
  bool use_graph_ = true;
  void apply_copy_writebacks(hipStream_t st);

  // GEMM lowering helpers
  bool gemm_desc(int i, tgk::GemmDesc& d) const;
  bool fold_into_producer(int perm_op, int a, int out, const std::vector<int64_t>& perm);
  bool gemm_operand(int t, int which, const Dims& op_shape, bool batched, int64_t& M, int64_t& K, int64_t& batch,
                    int64_t& bdiv, int64_t& s0, int64_t& s1, int64_t& sr, int64_t& sc, bool transposeOk) const;
  void add_node(Node n) { nodes_.push_back(std::move(n)); }
  void lower_op(int i);

  // GEMMs whose results only the fused optimizer reads (weight gradients) and that would
  // split K run together just before it: one grouped launch per operand-layout kind, with
  // whole-K tiles, instead of one launch plus a split-K reduction each.
  struct DeferredGemm { int op; tgk::GemmDesc d; int a, b, out, kind; };
  std::vector<DeferredGemm> deferred_gemms_;
  std::vector<char> defer_gemm_;     // op -> runs in a grouped launch
  // Fused optimizer (k_optim.hip). Per parameter: the update (adam_update_m / _v / _p, or
  // the pointwise chain of src/sgd.ts:155-170) and the gradient transforms ahead of it
  // (normalizeGrads: g / broadcast(norm), clipGradNorm: g * broadcast(scale);
  // src/grad.ts:110-172) run in one update launch. The transforms' scalars come from
  // grad_norms launches just before it: per-parameter sums of squares, then a scalar
  // program restating the IR's rank-0 ops (chained adds, sqrt, add_scalar, div, min).
  struct OptParam {
    int p = -1, g = -1;          // param tensor; gradient as the backward pass leaves it
    int final_g = -1;            // the gradient tensor the update reads in the IR
    int gdiv = -1, gmul = -1;    // transform scalar tensors (-1: none)
    int div_out = -1;            // the normalised gradient tensor (output of the div)
    int m = -1, v = -1;          // Adam moments; SGD: m = velocity
    int lr = -1;                 // lrt (Adam) / lr (SGD) tensor
    int shrink_t = -1;           // Adam: per-step decay shrink tensor
    double shrink = 1.0;         // Adam: static decay shrink; SGD: weight decay
    double mom = 0.0;            // SGD momentum
    int flags = 0;               // SGD: 1 Nesterov, 2 weight decay, 4 momentum
  };
  std::vector<OptParam> opt_params_;
  bool opt_sgd_ = false;
  tgk::AdamHyper opt_hyper_{0.9, 0.1, 0.999, 0.001, 1e-8};
  std::set<int> adam_ops_;           // IR ops the fused optimizer executes (updates and transforms)
  struct NormSum { int g, pre_t, launch; };       // f32 sum of squares of g (divided by scalar pre_t first)
  std::vector<NormSum> norm_sums_;
  std::vector<int> norm_sum_val_;                  // value index of each sum
  std::map<int, int> norm_val_;                    // scalar tensor -> value index
  std::vector<tgk::ScalarInstr> norm_prog_[2];     // scalar program per norm launch
  int norm_nvals_ = 0, norm_launches_ = 0;
  bool use_fused_transforms_ = true;               // TG_OPT_FUSED=0: transforms and SGD op by op
  void match_optimizer();
  bool match_sgd(int pnew, const std::string& name, const std::map<std::string, int>& state_wb, OptParam& q,
                 std::set<int>& ops, std::set<int>& wb) const;
  bool scalar_bcast(int t) const;
  bool opt_closed(const std::set<int>& ops, const std::set<int>& wb_ok) const;
  void match_grad_transforms();
  void emit_optimizer();
  void plan_gemm_groups();
  // A GEMM whose product only one element-form group reads (contiguously, in its own
  // iteration order) can run that group in its epilogue: one launch instead of two, and
  // the product never reaches memory. By default only groups of inexpensive ops (adds,
  // products, relu and the like; C4's bias + relu layers: 385 -> 393 steps/s): a group with
  // f64 transcendentals or the dropout hash runs them on the GEMM's eight wavefronts per CU
  // after the matrix work instead of beside other work, which measured slower (C5's GELU,
  // C2's tanh). TG_GEMM_EPI=1 takes every group the epilogue can run, 0 none.
  enum { kEpiOff = 0, kEpiAll = 1, kEpiCheap = 2 };
  int gemm_epi_mode_ = kEpiCheap;
  bool epi_cheap(int gi) const;
  std::vector<char> group_done_;     // group already run inside a GEMM epilogue
  int epi_group(int op, int out, const tgk::GemmDesc& d, bool& store_c, const CatFwd* cat = nullptr) const;
  void lower_gemm_epi(int op, const tgk::GemmDesc& d, int a, int b, int out, int gi, bool store_c,
                      const CatFwd* cat = nullptr);
  // Column sums read only by the optimizer (bias, LayerNorm gain / shift gradients) run
  // together with the grouped GEMMs, kColSumMax per launch.
  std::vector<char> defer_colsum_;
  void emit_colsums(const std::vector<int>& batch, bool with_scatter = false, bool with_rowsums = false,
                    bool with_mids = false);
  // A row group that only reduces one row to a scalar the graph outputs (the loss mean:
  // sum_last or mean_last, then optionally mul_scalar) runs as a one-column sum in the first
  // deferred column-sum launch (TG_COLSUM_LOSS=0: a launch of its own in place).
  struct DeferredRowSum { int gi, a, out; int64_t R; double div, scale; std::string detail; };
  // Sums over the outer and inner axes of a contiguous [B, C, L] array that only the
  // optimizer reads (convolution bias gradients) run in the same launch (TG_COLSUM_MID=0:
  // as their own reductions in place).
  struct DeferredMidSum { int a, out; int64_t B, C, L; };
  std::vector<DeferredMidSum> deferred_midsum_;
  bool use_colsum_mid_ = true;
  bool any_deferred_colsum_ = false;
  std::vector<DeferredRowSum> deferred_rowsum_;
  bool use_colsum_loss_ = true;
  bool tail_rowsum(int gi, DeferredRowSum& d) const;
  // An embedding gradient (sort-free scatter form) that only the optimizer reads runs in the
  // first deferred column-sum launch, its blocks ahead of the sums' (TG_COLSUM_SCATTER=0:
  // a launch of its own in place).
  struct DeferredScatter { int op, idx, b, out; int64_t rows, V, N; std::string shape; };
  std::vector<DeferredScatter> deferred_scatter_;
  bool use_colsum_scatter_ = true;
  void emit_scatter(const DeferredScatter& sc);
  bool use_gemm_group_ = true;       // TG_GEMM_GROUP=0 keeps every GEMM in place
  bool use_remat_ = true;            // TG_REMAT=0 stores every value another group reads
  bool only_optimizer_reads(int t) const;
  void flush_deferred_gemms();
  void emit_gemm_group(const std::vector<DeferredGemm>& grp);
  // Independent GEMMs whose own plan is a single-pass 64 x 64 tiling (few tiles each) and
  // whose operands are ready share one grouped launch at the first one's position.
  std::vector<char> gemm_done_;      // op already emitted inside an earlier group
  bool plain_gemm(int j) const;
  bool ready_now(int t) const;
  void check_gemm_spans(const tgk::GemmDesc& d, int a, int b, int out) const;
  std::vector<void*> dev_tables_;    // device copies of grouped-launch tables
};

// ---------------------------------------------------------------------------------------

Runtime::Runtime(const char* json, Runtime* par, bool plan_only) : parent(par) {
  if (const char* g = std::getenv("TG_GRAPH")) use_graph_ = std::string(g) != "0";
  if (const char* g = std::getenv("TG_GEMM_GROUP")) use_gemm_group_ = std::string(g) != "0";
  if (const char* g = std::getenv("TG_GEMM_SUM")) use_gemm_sum_ = std::string(g) != "0";
  if (const char* g = std::getenv("TG_REMAT")) use_remat_ = std::string(g) != "0";
  if (const char* g = std::getenv("TG_COLSUM_SCATTER")) use_colsum_scatter_ = std::string(g) != "0";
  if (const char* g = std::getenv("TG_COLSUM_LOSS")) use_colsum_loss_ = std::string(g) != "0";
  if (const char* g = std::getenv("TG_COLSUM_MID")) use_colsum_mid_ = std::string(g) != "0";
  if (const char* g = std::getenv("TG_COLSUM_EPI")) use_colsum_epi_ = std::string(g) != "0";
  if (const char* g = std::getenv("TG_GEMM_EPI")) gemm_epi_mode_ = std::string(g) == "1" ? kEpiAll : (std::string(g) == "0" ? kEpiOff : kEpiCheap);
  if (const char* g = std::getenv("TG_FUSED")) use_jit_ = std::string(g) != "vm";
  if (const char* g = std::getenv("TG_CONV")) use_conv_gemm_ = std::string(g) != "direct";
  // A several-stream schedule of the step was tried and crashed inside the HIP runtime
  // while capturing the transformer step; it is removed, and asking for it is an error.
  if (const char* g = std::getenv("TG_STREAMS"))
    if (std::string(g) != "1")
      throw Error(TG_INVALID_ARGUMENT, "TG_STREAMS: only one stream per step is supported");
  try {
    doc_ = tgj::parse(json);
  } catch (std::exception& e) {
    throw Error(TG_INVALID_ARGUMENT, e.what());
  }
  // A document missing fields or holding values of the wrong type is the caller's error.
  try {
    read_document();
  } catch (Error&) {
    throw;
  } catch (std::exception& e) {
    throw Error(TG_INVALID_ARGUMENT, std::string("IR: ") + e.what());
  }
  plan_only_ = plan_only;
  analyse();
  relu_grads_from_outputs();
  narrow_sliced_products();
  compute_views();
  lower();
  if (!plan_only) hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
  split_init_nodes();
  allocate();
  bind_all();   // in plan-only mode this still runs every launch's host-side bounds proof
  jit_finish();
  if (!plan_only) prepare_noalloc();
  if (!plan_only && !init_nodes_.empty()) {
    for (auto& n : init_nodes_) n.launch(stream_);
    hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize(constants)");
  }
}

// Tensors, ops, outputs, captures and the optimizer block of the IR document.
void Runtime::read_document() {
  const tgj::Value& g = doc_.at("graph");
  for (const auto& t : g.at("tensors").items) {
    TInfo ti;
    for (const auto& d : t.at("shape").items) ti.shape.push_back(d.i64());
    ti.dt = parse_dt(t.at("dtype").str());
    ti.numel = prod(ti.shape);
    ti.src = -1;
    T_.push_back(ti);
  }
  for (const auto& op : g.at("ops").items) {
    ops_.push_back(&op);
    kinds_.push_back(op.at("kind").str());
  }
  for (size_t i = 0; i < ops_.size(); ++i) {
    int out = ops_[i]->at("out").i32();
    if (out < 0 || out >= (int)T_.size()) throw Error(TG_INVALID_ARGUMENT, "IR: op output id out of range");
    T_[out].src = (int)i;
  }
  for (const auto& o : g.at("outputs").items) outputs_.push_back(o.i32());
  if (const tgj::Value* c = g.get("captures"))
    for (const auto& m : c->members) { captures_[m.first] = m.second.i32(); capture_names.push_back(m.first); }
  if (const tgj::Value* opt = doc_.get("optimizer"))
    if (!opt->null()) {
      opt_kind_ = opt->at("kind").str();
      opt_cfg_ = &opt->at("config");
      lr_ = opt_cfg_->at("lr");
    }
  if (parent && opt_cfg_) throw Error(TG_INVALID_ARGUMENT, "compileForward: a sibling graph cannot carry an optimizer");
}

Runtime::~Runtime() {
  if (graph_exec_) hipGraphExecDestroy(graph_exec_);
  if (graph_) hipGraphDestroy(graph_);
  if (stream_) { hipStreamSynchronize(stream_); hipStreamDestroy(stream_); }
  if (arena_) hipFree(arena_);
  if (input_region_) hipFree(input_region_);
  if (workspace_ && !plan_only_) hipFree(workspace_);
  if (counters_ && !plan_only_) hipFree(counters_);
  if (partials_ && !plan_only_) hipFree(partials_);
  if (fused_code_dev_ && !plan_only_) hipFree(fused_code_dev_);
  for (void* t : dev_tables_) hipFree(t);
  for (char* p : slots_) if (p) hipFree(p);
  if (staging_) hipHostFree(staging_);
  if (loss_host_) hipHostFree(loss_host_);
}

// Op -> input tensor ids, canonical order (src/ir.ts:356-395).
static std::vector<int> op_inputs(const tgj::Value& op) {
  static const std::map<std::string, std::vector<const char*>> F = {
      {"randn", {"seed"}}, {"dropout", {"a", "seed"}}, {"categorical_last", {"a", "seed"}},
      {"one_hot", {"indices"}}, {"where", {"cond", "a", "b"}}, {"relu_grad", {"x", "dy"}},
      {"adam_update_m", {"m", "g"}}, {"adam_update_v", {"v", "g"}},
      {"adam_update_p", {"p", "mNew", "vNew", "lrt", "decayShrinkTensor"}},
      {"conv2d", {"input", "weight"}}, {"conv2d_input_grad", {"weight", "dy"}},
      {"conv2d_weight_grad", {"input", "dy"}}, {"max_pool_2d", {"input"}},
      {"max_pool_2d_grad", {"input", "dy"}},
      {"param_input", {}}, {"tensor_input", {}}, {"state_input", {}}, {"arange", {}},
      {"const_scalar", {}}, {"const_fill", {}},
  };
  const std::string& k = op.at("kind").str();
  std::vector<int> ids;
  if (k == "concat") {
    for (const auto& x : op.at("inputs").items) ids.push_back(x.i32());
    return ids;
  }
  auto it = F.find(k);
  if (it != F.end()) {
    for (const char* f : it->second) {
      const tgj::Value& v = op.at(f);
      if (!v.null()) ids.push_back(v.i32());
    }
    return ids;
  }
  if (op.get("b")) { ids.push_back(op.at("a").i32()); ids.push_back(op.at("b").i32()); return ids; }
  ids.push_back(op.at("a").i32());
  return ids;
}

void Runtime::analyse() {
  consumers_.assign(T_.size(), {});
  for (size_t i = 0; i < ops_.size(); ++i) {
    for (int id : op_inputs(*ops_[i])) {
      if (id < 0 || id >= (int)T_.size()) throw Error(TG_INVALID_ARGUMENT, "IR: op input id out of range");
      consumers_[id].push_back((int)i);
    }
    const std::string& k = kinds_[i];
    int out = ops_[i]->at("out").i32();
    if (k == "param_input") {
      const std::string& nm = ops_[i]->at("name").str();
      param_names.push_back(nm);
      param_root[nm] = out;
    } else if (k == "tensor_input") {
      input_tid_[ops_[i]->at("name").str()] = out;
      if (ops_[i]->at("name").str() == "__prngSeed") uses_prng_ = true;
    } else if (k == "state_input") {
      state_tid_[ops_[i]->at("name").str()] = out;
    }
  }
  for (auto& kv : state_tid_) state_list_.push_back(kv.first);
}

// relu_grad(x, dy) = x > 0 ? dy : 0 reads the pre-activation x. Where relu(x) is also
// computed, relu(x) > 0 exactly when x > 0 (NaN and -0 included: relu maps them to values
// that are not > 0), so the gradient reads the relu output instead: the output is kept
// for the next layer anyway, and the pre-activation then need not be stored at all (an
// add + relu group writes one [rows, width] tensor instead of two). The IR document is
// rewritten in place; every value stays bit-identical.
void Runtime::relu_grads_from_outputs() {
  for (size_t i = 0; i < ops_.size(); ++i) {
    if (kinds_[i] != "relu_grad") continue;
    const int x = fld((int)i, "x");
    if (T_[x].dt != F32) continue;
    int r = -1;
    for (int c : consumers_[x])
      if (c < (int)i && kinds_[c] == "relu" && fld(c, "a") == x) { r = O(c).at("out").i32(); break; }
    if (r < 0 || T_[r].shape != T_[x].shape || T_[r].dt != F32) continue;
    const_cast<tgj::Value&>(ops_[i]->at("x")).number = (double)r;
    auto& cx = consumers_[x];
    cx.erase(std::find(cx.begin(), cx.end(), (int)i));
    consumers_[r].push_back((int)i);
    std::sort(consumers_[r].begin(), consumers_[r].end());
  }
}

// A product read only by a slice that keeps its first columns (the input gradient of a
// concatenation's first part): the GEMM computes only those columns, reading the first
// N' columns of B through the same view, and the slice, which then covers the whole
// (narrowed) product, becomes a view of it in compute_views. The IR shape of the product
// is rewritten in place; every kept element is the same dot product as before.
void Runtime::narrow_sliced_products() {
  auto pinned = [&](int t) {
    for (int o : outputs_) if (o == t) return true;
    for (auto& c : captures_) if (c.second == t) return true;
    if (const tgj::Value* wbs = doc_.get("writebacks"))
      for (const auto& w : wbs->items) if (w.at("source").i32() == t) return true;
    return false;
  };
  for (size_t j = 0; j < ops_.size(); ++j) {
    if (kinds_[j] != "slice_range") continue;
    const int p = fld((int)j, "a"), s = O((int)j).at("out").i32();
    const int m = T_[p].src;
    if (m < 0 || (kinds_[m] != "matmul" && kinds_[m] != "matmul_batched") || T_[p].dt != F32) continue;
    if (consumers_[p].size() != 1 || pinned(p)) continue;
    // products of a one-hot (the embedding gather and scatter) read B's rows whole
    const int am = T_[fld(m, "a")].src;
    if (am >= 0 && (kinds_[am] == "one_hot" || kinds_[am] == "permute" || kinds_[am] == "reshape")) {
      int r = am;
      while (r >= 0 && (kinds_[r] == "permute" || kinds_[r] == "reshape")) r = T_[fld(r, "a")].src;
      if (r >= 0 && kinds_[r] == "one_hot") continue;
    }
    Dims& ps = T_[p].shape;
    const Dims& ss = T_[s].shape;
    const int64_t rank = (int64_t)ps.size();
    int64_t ax = O((int)j).at("axis").i64();
    if (ax < 0) ax += rank;
    if (rank < 2 || ax != rank - 1 || O((int)j).at("start").i64() != 0 || ss.size() != ps.size()) continue;
    if (!std::equal(ps.begin(), ps.end() - 1, ss.begin()) || ss.back() <= 0 || ss.back() >= ps.back()) continue;
    ps.back() = ss.back();
    T_[p].numel = prod(ps);
  }
}

// Views: every tensor is (root storage, dims, strides). Aliasing ops inherit their
// input's root; permutes are strided views until a consumer needs contiguous data.
// A permute that must be materialised, applied to the fresh output of a GEMM read by
// nothing else (directly, or through one permuting view that is itself read only by this
// permute): let the GEMM write the permuted layout directly. The permute's output becomes
// the storage root and the GEMM output a strided view of it, so no copy runs.
bool Runtime::fold_into_producer(int perm_op, int a, int out, const std::vector<int64_t>& perm) {
  const int g = view_[a].root;
  const int src = T_[g].src;
  if (src < 0 || (kinds_[src] != "matmul" && kinds_[src] != "matmul_batched")) return false;
  if (O(src).at("out").i32() != g || !view_[g].contiguous() || view_[g].root != g) return false;
  if (consumers_[a].size() != 1 || consumers_[a][0] != perm_op) return false;
  auto pinned = [&](int t) {
    for (int o : outputs_) if (o == t) return true;
    for (auto& c : captures_) if (c.second == t) return true;
    if (const tgj::Value* wbs = doc_.get("writebacks"))
      for (const auto& w : wbs->items) if (w.at("source").i32() == t) return true;
    return false;
  };
  if (pinned(a) || pinned(g)) return false;
  // a == g, or a is a permutation view of g: each dim of a is one dim of g.
  const Dims cg = contiguous_strides(T_[g].shape);
  std::vector<int> dim_of_g(T_[a].shape.size(), -1);   // a's dim e -> g's dim
  if (a != g) {
    if (consumers_[g].size() != 1 || kinds_[consumers_[g][0]] != "permute" ||
        O(consumers_[g][0]).at("out").i32() != a)
      return false;
    const View& v = view_[a];
    if (v.dims.size() != T_[g].shape.size()) return false;
    std::vector<bool> used(cg.size(), false);
    for (size_t e = 0; e < v.dims.size(); ++e) {
      for (size_t q = 0; q < cg.size(); ++q)
        if (!used[q] && T_[g].shape[q] == v.dims[e] && (cg[q] == v.strides[e] || v.dims[e] == 1)) {
          used[q] = true;
          dim_of_g[e] = (int)q;
          break;
        }
      if (dim_of_g[e] < 0) return false;
    }
  } else {
    for (size_t e = 0; e < dim_of_g.size(); ++e) dim_of_g[e] = (int)e;
  }
  const Dims cs = contiguous_strides(T_[out].shape);
  View va{out, T_[a].shape, Dims(T_[a].shape.size(), 0)};
  for (size_t d = 0; d < perm.size(); ++d) va.strides[perm[d]] = cs[d];
  View vg{out, T_[g].shape, Dims(T_[g].shape.size(), 0)};
  for (size_t e = 0; e < dim_of_g.size(); ++e) vg.strides[dim_of_g[e]] = va.strides[e];
  const View saved_g = view_[g], saved_a = view_[a];
  view_[g] = vg;
  view_[a] = va;
  tgk::GemmDesc d{};
  if (!gemm_desc(src, d)) {
    view_[g] = saved_g;
    view_[a] = saved_a;
    return false;
  }
  view_[out] = View{out, T_[out].shape, cs};
  return true;
}

void Runtime::compute_views() {
  const size_t n = T_.size();
  view_.resize(n);
  virtual_.assign(ops_.size(), false);
  materialize_.assign(n, false);
  for (size_t t = 0; t < n; ++t) view_[t] = View{(int)t, T_[t].shape, contiguous_strides(T_[t].shape)};

  // Leading (batch) dims of a GEMM operand view must merge into at most two strided
  // dims for the kernel's two-level batch index.
  auto gemm_view_ok = [&](const View& v) {
    if (v.dims.size() < 2) return false;
    Dims d3, s3;
    for (size_t i = 0; i + 2 < v.dims.size(); ++i) {
      if (v.dims[i] == 1) continue;
      if (!d3.empty() && s3.back() == v.strides[i] * v.dims[i]) { d3.back() *= v.dims[i]; s3.back() = v.strides[i]; }
      else { d3.push_back(v.dims[i]); s3.push_back(v.strides[i]); }
    }
    return d3.size() <= 2;
  };
  auto consumer_needs_contiguous = [&](int t, const View& v) {
    for (int c : consumers_[t]) {
      const std::string& k = kinds_[c];
      if (k == "permute") continue;   // composes strides
      if (k == "matmul" || k == "matmul_batched") {
        if (!gemm_view_ok(v)) return true;
        continue;
      }
      if (k == "add" || k == "sub" || k == "mul" || k == "div" || k == "min" || k == "max" || k == "less" ||
          k == "greater" || k == "broadcast_to")
        continue;   // strided element-wise kernels
      return true;
    }
    for (int o : outputs_) if (o == t) return true;
    for (auto& c : captures_) if (c.second == t) return true;
    return false;
  };

  // n if tensor t reads the n x n identity one_hot(arange(n), n) as laid out or transposed,
  // else -1 (position embeddings: one_hot(arange(T)) @ table and its gradient).
  auto identity_onehot = [&](int t) -> int64_t {
    const int r = view_[t].root;
    const int src = T_[r].src;
    if (src < 0 || kinds_[src] != "one_hot" || T_[r].dt != F32) return -1;
    const int idx = fld(src, "indices");
    const int isrc = T_[view_[idx].root].src;
    const int64_t n = O(src).at("depth").i64();
    if (isrc < 0 || kinds_[isrc] != "arange" || T_[idx].numel != n || !view_[idx].contiguous()) return -1;
    const View& v = view_[t];
    if (v.dims.size() != 2 || v.dims[0] != n || v.dims[1] != n) return -1;
    if (!((v.strides[0] == n && v.strides[1] == 1) || (v.strides[0] == 1 && v.strides[1] == n))) return -1;
    return n;
  };

  for (size_t i = 0; i < ops_.size(); ++i) {
    const std::string& k = kinds_[i];
    int out = ops_[i]->at("out").i32();
    if (k == "matmul") {
      // identity(n) @ B = B: the product is B itself (a view, no kernel).
      const int a = ops_[i]->at("a").i32(), b = ops_[i]->at("b").i32();
      const int64_t n = identity_onehot(a);
      if (n > 0 && view_[b].contiguous() && T_[b].shape.size() == 2 && T_[b].shape[0] == n &&
          T_[out].numel == T_[b].numel) {
        view_[out] = View{view_[b].root, T_[out].shape, contiguous_strides(T_[out].shape)};
        virtual_[i] = true;
      }
    } else if (k == "reshape" || k == "stop_gradient") {
      int a = ops_[i]->at("a").i32();
      const View& va = view_[a];
      if (va.contiguous()) {
        view_[out] = View{va.root, T_[out].shape, contiguous_strides(T_[out].shape)};
        virtual_[i] = true;
      }
    } else if (k == "slice_range" && T_[ops_[i]->at("a").i32()].shape == T_[out].shape &&
               ops_[i]->at("start").i64() == 0) {
      // a slice covering its whole input (a narrowed product's)
      int a = ops_[i]->at("a").i32();
      if (view_[a].contiguous()) {
        view_[out] = View{view_[a].root, T_[out].shape, contiguous_strides(T_[out].shape)};
        virtual_[i] = true;
      }
    } else if ((k == "sum_to_shape" || k == "broadcast_to") &&
               T_[ops_[i]->at("a").i32()].shape == T_[out].shape) {
      int a = ops_[i]->at("a").i32();
      if (view_[a].contiguous()) {
        view_[out] = View{view_[a].root, T_[out].shape, contiguous_strides(T_[out].shape)};
        virtual_[i] = true;
      }
    } else if (k == "permute") {
      int a = ops_[i]->at("a").i32();
      const View& va = view_[a];
      std::vector<int64_t> perm;
      for (const auto& p : ops_[i]->at("perm").items) perm.push_back(p.i64());
      View v{va.root, {}, {}};
      for (size_t d = 0; d < perm.size(); ++d) {
        v.dims.push_back(va.dims[perm[d]]);
        v.strides.push_back(va.strides[perm[d]]);
      }
      if (!consumer_needs_contiguous(out, v) && !v.contiguous()) {
        view_[out] = v;
        virtual_[i] = true;
      } else if (v.contiguous()) {
        view_[out] = View{va.root, T_[out].shape, contiguous_strides(T_[out].shape)};
        virtual_[i] = true;
      } else if (fold_into_producer(i, a, out, perm)) {
        virtual_[i] = true;
      } else {
        materialize_[out] = true;
      }
    }
  }
}

// Express operand `t` of a GEMM as [batch, rows, cols] with rows/cols strides and a
// two-level batch decomposition. `op_shape` is the IR shape of the operand.
bool Runtime::gemm_operand(int t, int which, const Dims& op_shape, bool batched, int64_t& R, int64_t& C,
                           int64_t& batch, int64_t& bdiv, int64_t& s0, int64_t& s1, int64_t& sr, int64_t& sc,
                           bool) const {
  (void)which;
  const View& v = view_[t];
  const int r = (int)v.dims.size();
  R = v.dims[r - 2];
  C = v.dims[r - 1];
  sr = v.strides[r - 2];
  sc = v.strides[r - 1];
  // leading dims
  Dims ld(v.dims.begin(), v.dims.end() - 2), ls(v.strides.begin(), v.strides.end() - 2);
  // drop size-1 dims
  Dims d2, s2;
  for (size_t i = 0; i < ld.size(); ++i) if (ld[i] != 1) { d2.push_back(ld[i]); s2.push_back(ls[i]); }
  // merge adjacent dims with compatible strides
  Dims d3, s3;
  for (size_t i = 0; i < d2.size(); ++i) {
    if (!d3.empty() && s3.back() == s2[i] * d2[i]) { d3.back() *= d2[i]; s3.back() = s2[i]; }
    else { d3.push_back(d2[i]); s3.push_back(s2[i]); }
  }
  (void)op_shape;
  (void)batched;
  batch = prod(d3);
  if (d3.size() == 0) { bdiv = 1; s0 = 0; s1 = 0; return true; }
  if (d3.size() == 1) { bdiv = 1; s0 = s3[0]; s1 = 0; return true; }
  if (d3.size() == 2) { bdiv = d3[1]; s0 = s3[0]; s1 = s3[1]; return true; }
  return false;
}

// Readers of a last-axis concatenation X = [S0 | S1] ([R, k0 + k1], f32, contiguous
// sources): a product reading X as its A operand (a layer fed by a skip connection) runs
// as one GEMM over the two sources when S0 fills whole 32-k stages (tgk::gemm_cat); a
// product reading X's transpose runs one GEMM per source (the weight gradient, in
// lower_op). When every reader (through reshape / permute views) is one of these, X itself
// is never written.
void Runtime::match_concat_products() {
  cat_fwd_.clear();
  cat_absorbed_.assign(ops_.size(), 0);
  if (!use_gemm_group_) return;
  auto pinned = [&](int t) {
    for (int o : outputs_) if (root(o) == root(t)) return true;
    for (auto& c : captures_) if (root(c.second) == root(t)) return true;
    for (auto& w : copy_writebacks_) if (root(w.first) == root(t)) return true;
    return false;
  };
  for (size_t c = 0; c < ops_.size(); ++c) {
    if (kinds_[c] != "concat" || virtual_[c]) continue;
    const int x = O((int)c).at("out").i32();
    if (view_[x].root != x || !view_[x].contiguous() || T_[x].dt != F32 || T_[x].shape.size() != 2 || pinned(x))
      continue;
    int64_t ax = O((int)c).at("axis").i64();
    if (ax < 0) ax += 2;
    const auto& ins = O((int)c).at("inputs").items;
    if (ax != 1 || ins.size() != 2) continue;
    const int s0 = ins[0].i32(), s1 = ins[1].i32();
    const int64_t R = T_[x].shape[0], Kt = T_[x].shape[1];
    bool ok_src = true;
    for (int s : {s0, s1})
      ok_src = ok_src && T_[s].dt == F32 && T_[s].shape.size() == 2 && T_[s].shape[0] == R && view_[s].contiguous();
    if (!ok_src) continue;
    const CatFwd cf{s0, s1, T_[s0].shape[1], T_[s1].shape[1]};
    if (cf.k0 + cf.k1 != Kt) continue;
    // every reader, through views
    bool all = true;
    std::vector<int> fwd;
    std::vector<int> stack{x};
    while (!stack.empty() && all) {
      const int t = stack.back();
      stack.pop_back();
      for (int u : consumers_[t]) {
        const std::string& k = kinds_[u];
        if (virtual_[u] && (k == "reshape" || k == "permute" || k == "stop_gradient")) {
          stack.push_back(O(u).at("out").i32());
          continue;
        }
        if (k != "matmul" || virtual_[u] || fld(u, "b") == t) { all = false; break; }
        std::vector<int> srcs;
        std::vector<int64_t> offs;
        tgk::GemmDesc d{};
        if (!gemm_desc(u, d)) { all = false; break; }
        const View& va = view_[t];
        if (va.dims == Dims({R, Kt}) && va.strides == Dims({Kt, 1})) {
          d.sAm = cf.k0;
          d.A = reinterpret_cast<const float*>(uintptr_t(256));
          d.B = reinterpret_cast<const float*>(uintptr_t(256));
          if (!tgk::gemm_cat_ok(d, tgk::GemmCat{reinterpret_cast<const float*>(uintptr_t(256)), cf.k0, cf.k1})) {
            all = false;
            break;
          }
          fwd.push_back(u);
        } else if (!(concat_transposed(t, srcs, offs) && !defer_gemm_[u] && d.batch == 1 && d.sCn == 1 &&
                     d.sCm == d.N && view_[O(u).at("out").i32()].contiguous())) {
          all = false;
          break;
        }
      }
    }
    // the forward products take the sources either way; X is skipped when nothing else reads it
    for (int u : fwd) cat_fwd_[u] = cf;
    if (all && !fwd.empty()) cat_absorbed_[c] = 1;
  }
}

void Runtime::check_cat_spans(const tgk::GemmDesc& d, const CatFwd& c, int b, int out, bool with_c) const {
  if (d.batch != 1 || d.K != c.k0 + c.k1 || d.sAm != c.k0 || d.sAk != 1)
    throw Error(TG_INTERNAL, "gemm_cat: descriptor does not match its sources");
  const int64_t da0[2] = {d.M, c.k0}, sa0[2] = {c.k0, 1};
  const int64_t da1[2] = {d.M, c.k1}, sa1[2] = {c.k1, 1};
  const int64_t db[2] = {d.K, d.N}, sb[2] = {d.sBk, d.sBn};
  const int64_t dc[2] = {d.M, d.N}, sc[2] = {d.sCm, d.sCn};
  check_span("gemm_cat A0", T_[root(c.src0)].numel, 0, da0, sa0, 2);
  check_span("gemm_cat A1", T_[root(c.src1)].numel, 0, da1, sa1, 2);
  check_span("gemm_cat B", T_[root(b)].numel, 0, db, sb, 2);
  if (with_c) check_span("gemm_cat C", T_[root(out)].numel, 0, dc, sc, 2);
  if (d.M * d.N != T_[out].numel) throw Error(TG_INTERNAL, "gemm_cat: output size mismatch");
}

// View t is the transpose [K0 + K1 + ..., R] of a concatenation along the last axis of
// contiguous f32 sources [R, K_s], each at least one 32-row MFMA block wide (narrower
// sources would each run a mostly empty tile): the sources and their first rows in the
// transpose.
bool Runtime::concat_transposed(int t, std::vector<int>& srcs, std::vector<int64_t>& offs) const {
  srcs.clear();
  offs.clear();
  const View& v = view_[t];
  const int x = v.root;
  const int c = T_[x].src;
  if (c < 0 || kinds_[c] != "concat" || virtual_[c] || T_[x].dt != F32 || T_[x].shape.size() != 2) return false;
  int64_t ax = O(c).at("axis").i64();
  if (ax < 0) ax += 2;
  const int64_t R = T_[x].shape[0], Kt = T_[x].shape[1];
  if (ax != 1 || v.dims != Dims({Kt, R}) || v.strides != Dims({1, Kt}) || !view_[x].contiguous()) return false;
  int64_t off = 0;
  for (const auto& e : O(c).at("inputs").items) {
    const int s = e.i32();
    if (T_[s].dt != F32 || T_[s].shape.size() != 2 || T_[s].shape[0] != R || T_[s].shape[1] < 32 ||
        !view_[s].contiguous())
      return false;
    srcs.push_back(s);
    offs.push_back(off);
    off += T_[s].shape[1];
  }
  return off == Kt && srcs.size() >= 2;
}

// Shapes and element strides of matmul op i as a GemmDesc (no pointers): operands read
// through their views (transposes and head permutes in place), the output written
// through its view (contiguous, or a permuted layout folded in by compute_views).
// Returns false if some view does not fit the kernel's two-level batch index.
bool Runtime::gemm_desc(int i, tgk::GemmDesc& d) const {
  const tgj::Value& op = O(i);
  const bool batched = kinds_[i] == "matmul_batched";
  const int a = op.at("a").i32(), b = op.at("b").i32(), out = op.at("out").i32();
  const Dims& ash = T_[a].shape;
  const Dims& bsh = T_[b].shape;
  // N from the product: a narrowed product reads only the first N columns of B
  const int64_t M = ash[ash.size() - 2], K = ash.back(), N = T_[out].shape.back();
  if (N > bsh.back()) return false;
  int64_t Ra, Ca, ba, bda, sa0, sa1, sar, sac;
  int64_t Rb, Cb, bb, bdb, sb0, sb1, sbr, sbc;
  int64_t Rc, Cc, bc, bdc, sc0, sc1, scr, scc;
  if (!gemm_operand(a, 0, ash, batched, Ra, Ca, ba, bda, sa0, sa1, sar, sac, true)) return false;
  if (!gemm_operand(b, 1, bsh, batched, Rb, Cb, bb, bdb, sb0, sb1, sbr, sbc, true)) return false;
  if (!gemm_operand(out, 2, T_[out].shape, batched, Rc, Cc, bc, bdc, sc0, sc1, scr, scc, true)) return false;
  const bool c_contig = view_[out].contiguous();
  d = tgk::GemmDesc{};
  d.N = N; d.K = K;
  if (!batched) {
    // A [..., M, K] @ B [K, N]: fold A's leading dims into M when they are uniformly
    // strided with the rows (and C's are too); otherwise batch over them with B broadcast.
    if (ba == 1 || (bda == 1 && sa0 == M * sar && (c_contig || (bdc == 1 && sc0 == M * scr)))) {
      d.M = M * ba; d.batch = 1; d.bdiv = 1;
      d.sAz0 = d.sAz1 = 0;
      d.sCz0 = d.sCz1 = 0;
    } else {
      d.M = M; d.batch = ba; d.bdiv = bda;
      d.sAz0 = sa0; d.sAz1 = sa1;
      d.sCz0 = M * N * bda; d.sCz1 = M * N;
    }
    d.sAm = sar; d.sAk = sac;
    d.sBz0 = d.sBz1 = 0; d.sBk = sbr; d.sBn = sbc;
  } else {
    // Batch dims of A and B must decompose identically.
    if (ba != bb) return false;
    d.M = M; d.batch = ba;
    if (bda == bdb || ba == 1) {
      d.bdiv = bda;
      d.sAz0 = sa0; d.sAz1 = sa1; d.sBz0 = sb0; d.sBz1 = sb1;
    } else if (bda == 1 && bdb != 1) {
      // A collapsed to one batch dim; split it like B.
      d.bdiv = bdb;
      d.sAz0 = sa0 * bdb; d.sAz1 = sa0; d.sBz0 = sb0; d.sBz1 = sb1;
    } else if (bdb == 1 && bda != 1) {
      d.bdiv = bda;
      d.sAz0 = sa0; d.sAz1 = sa1; d.sBz0 = sb0 * bda; d.sBz1 = sb0;
    } else {
      return false;
    }
    d.sAm = sar; d.sAk = sac; d.sBk = sbr; d.sBn = sbc;
    d.sCz0 = M * N * d.bdiv; d.sCz1 = M * N;
  }
  d.sCm = N; d.sCn = 1;
  if (!c_contig) {
    // Output written in a permuted layout: rows / cols from its view, batch split like
    // the operands'.
    if (Rc != d.M || Cc != N) return false;
    d.sCm = scr; d.sCn = scc;
    if (d.batch > 1) {
      if (bc != d.batch) return false;
      if (bdc == d.bdiv) { d.sCz0 = sc0; d.sCz1 = sc1; }
      else if (bdc == 1) { d.sCz0 = sc0 * d.bdiv; d.sCz1 = sc0; }
      else if (d.bdiv == 1) {
        // operands collapsed to one batch dim: split them like C
        d.bdiv = bdc;
        d.sAz1 = d.sAz0; d.sAz0 *= bdc;
        d.sBz1 = d.sBz0; d.sBz0 *= bdc;
        d.sCz0 = sc0; d.sCz1 = sc1;
      } else {
        return false;
      }
    }
  }
  return true;
}

// t = broadcast_to(s) of an f32 scalar s (one element).
bool Runtime::scalar_bcast(int t) const {
  const int op = T_[t].src;
  if (op < 0 || kinds_[op] != "broadcast_to") return false;
  const int s = fld(op, "a");
  return T_[s].numel == 1 && T_[s].dt == F32;
}

// Every op of `ops` has its readers inside `ops` or the fused optimizer, and its output is
// no graph output, capture or writeback source (except the sources in `wb_ok`, which the
// fused update stores in place).
bool Runtime::opt_closed(const std::set<int>& ops, const std::set<int>& wb_ok) const {
  const tgj::Value* wbs = doc_.get("writebacks");
  for (int o : ops) {
    const int out = O(o).at("out").i32();
    for (int c : consumers_[out])
      if (!ops.count(c) && !adam_ops_.count(c)) return false;
    for (int x : outputs_) if (x == out) return false;
    for (auto& c : captures_) if (c.second == out) return false;
    if (wbs)
      for (const auto& w : wbs->items)
        if (w.at("source").i32() == out && !wb_ok.count(out)) return false;
  }
  return true;
}

// The update chain sgd.ts:155-170 emits for one parameter, from its new value back to the
// gradient: p' = sub(p, mul(broadcast_to(lr), u)); u = e, v' or add(e, mul_scalar(v', mu))
// (Nesterov); v' = add(mul_scalar(v, mu), e); e = g or add(g, mul_scalar(p, wd)).
bool Runtime::match_sgd(int pnew, const std::string& name, const std::map<std::string, int>& state_wb, OptParam& q,
                        std::set<int>& ops, std::set<int>& wb) const {
  auto src = [&](int t) { return t >= 0 && t < (int)T_.size() ? T_[t].src : -1; };
  auto is = [&](int op, const char* k) { return op >= 0 && kinds_[op] == k; };
  // x = mul_scalar(of, k) in either operand of a binary op: (other operand, mul_scalar op)
  auto scaled = [&](int bop, int of, int& other, int& ms) {
    for (int side = 0; side < 2; ++side) {
      const int x = fld(bop, side ? "a" : "b"), y = fld(bop, side ? "b" : "a");
      if (is(src(x), "mul_scalar") && fld(src(x), "a") == of) { other = y; ms = src(x); return true; }
    }
    return false;
  };
  auto ip = param_root.find(name);
  if (ip == param_root.end()) return false;
  const int p = ip->second;
  const int s = src(pnew);
  if (!is(s, "sub") || fld(s, "a") != p) return false;
  const int mo = src(fld(s, "b"));
  if (!is(mo, "mul")) return false;
  int bc = fld(mo, "a"), u = fld(mo, "b");
  if (!scalar_bcast(bc)) std::swap(bc, u);
  if (!scalar_bcast(bc)) return false;
  const int lr = fld(src(bc), "a");
  const tgj::Value* ln = opt_cfg_ ? opt_cfg_->get("lrInputName") : nullptr;
  if (!ln || ln->null() || !input_tid_.count(ln->str()) || input_tid_.at(ln->str()) != lr) return false;
  q = OptParam{};
  q.p = p;
  q.lr = lr;
  ops.insert({s, mo, src(bc)});
  wb.insert(pnew);
  int e = u;
  auto iv = state_wb.find("sgd_v_" + name);
  if (iv != state_wb.end()) {
    const int vn = iv->second;
    double mu2 = -1;
    if (u != vn) {
      const int na = src(u);
      int ms = -1;
      if (!is(na, "add") || !scaled(na, vn, e, ms)) return false;
      mu2 = O(ms).at("scalar").num();
      q.flags |= 1;
      ops.insert({na, ms});
    }
    const int va = src(vn);
    auto is_ = state_tid_.find("sgd_v_" + name);
    if (!is(va, "add") || is_ == state_tid_.end()) return false;
    int e2 = -1, ms = -1;
    if (!scaled(va, is_->second, e2, ms)) return false;
    q.mom = O(ms).at("scalar").num();
    if (q.flags & 1) {
      if (e2 != e || mu2 != q.mom) return false;
    } else {
      e = e2;
    }
    q.m = is_->second;
    q.flags |= 4;
    ops.insert({va, ms});
    wb.insert(vn);
  }
  const int ea = src(e);
  int g = e, ms = -1;
  if (is(ea, "add") && scaled(ea, p, g, ms)) {
    q.shrink = O(ms).at("scalar").num();
    q.flags |= 2;
    ops.insert({ea, ms});
  } else {
    g = e;
  }
  if (T_[g].numel != T_[p].numel || T_[g].dt != F32) return false;
  q.final_g = q.g = g;
  return true;
}

void Runtime::match_optimizer() {
  opt_params_.clear();
  adam_ops_.clear();
  opt_sgd_ = false;
  std::set<int> fused_wb;
  std::vector<int> adam_p_ops;
  for (size_t i = 0; i < ops_.size(); ++i) if (kinds_[i] == "adam_update_p") adam_p_ops.push_back((int)i);
  for (int pi : adam_p_ops) {
    const int mNew = fld(pi, "mNew"), vNew = fld(pi, "vNew"), p = fld(pi, "p");
    const int mo = T_[mNew].src, vo = T_[vNew].src;
    if (kinds_[mo] != "adam_update_m" || kinds_[vo] != "adam_update_v" || kinds_[T_[p].src] != "param_input" ||
        kinds_[T_[fld(mo, "m")].src] != "state_input" || kinds_[T_[fld(vo, "v")].src] != "state_input")
      throw Error(TG_INVALID_ARGUMENT, "IR: adam_update_p is not fed by adam_update_m/v of state inputs");
    if (fld(mo, "g") != fld(vo, "g"))
      throw Error(TG_INVALID_ARGUMENT, "IR: adam_update_m and adam_update_v read different gradients");
    OptParam q;
    q.p = p;
    q.m = fld(mo, "m");
    q.v = fld(vo, "v");
    q.final_g = q.g = fld(mo, "g");
    q.lr = fld(pi, "lrt");
    const tgj::Value& ds = O(pi).at("decayShrinkTensor");
    q.shrink_t = ds.null() ? -1 : ds.i32();
    q.shrink = ds.null() ? O(pi).at("decayShrink").num() : 1.0;
    const double b1 = O(mo).at("beta1").num(), b2 = O(vo).at("beta2").num();
    opt_hyper_ = {b1, 1 - b1, b2, 1 - b2, O(pi).at("eps").num()};
    if (!opt_params_.empty() && opt_params_.front().lr != q.lr)
      throw Error(TG_INVALID_ARGUMENT, "IR: adam_update_p ops read different lrt tensors");
    opt_params_.push_back(q);
    adam_ops_.insert({pi, mo, vo});
    fused_wb.insert({O(pi).at("out").i32(), mNew, vNew});
  }
  const tgj::Value* wbs = doc_.get("writebacks");
  if (adam_p_ops.empty() && opt_kind_ == "sgd" && wbs && use_fused_transforms_) {
    // every parameter's update must be the SGD chain; otherwise all of it runs op by op
    std::map<std::string, int> state_wb;
    for (const auto& w : wbs->items)
      if (w.at("destKind").str() == "state") state_wb[w.at("destName").str()] = w.at("source").i32();
    std::vector<OptParam> qs;
    std::set<int> ops, wb;
    bool ok = true;
    for (const auto& w : wbs->items) {
      if (w.at("destKind").str() != "param") continue;
      OptParam q;
      if (!match_sgd(w.at("source").i32(), w.at("destName").str(), state_wb, q, ops, wb) ||
          (!qs.empty() && qs.front().lr != q.lr)) {
        ok = false;
        break;
      }
      qs.push_back(q);
    }
    if (ok && !qs.empty() && opt_closed(ops, wb)) {
      opt_params_ = qs;
      adam_ops_ = ops;
      fused_wb = wb;
      opt_sgd_ = true;
    }
  }
  if (wbs)
    for (const auto& w : wbs->items) {
      const int src = w.at("source").i32();
      if (fused_wb.count(src)) continue;
      copy_writebacks_.emplace_back(src, w.at("destName").str());
    }
  if (!opt_params_.empty() && use_fused_transforms_) match_grad_transforms();
}

// normalizeGrads (grad.ts:148-172) and clipGradNorm (grad.ts:110-130) in front of the
// fused update: per parameter, g_final = mul(div(g, broadcast(norm)), broadcast(scale))
// with either layer optional. Their scalars must be computable from per-parameter sums of
// squares (sum_last(reshape(mul(y, y)))) of the gradients or the normalised gradients, and
// constants, by rank-0 ops; and nothing else may read any of the absorbed values.
// Otherwise the transforms run op by op and the update reads their result.
void Runtime::match_grad_transforms() {
  auto src = [&](int t) { return t >= 0 && t < (int)T_.size() ? T_[t].src : -1; };
  auto is = [&](int op, const char* k) { return op >= 0 && kinds_[op] == k; };
  std::set<int> ops;
  bool any = false;
  for (OptParam& q : opt_params_) {
    int t = q.final_g;
    const int mo = src(t);
    if (is(mo, "mul")) {
      int a = fld(mo, "a"), b = fld(mo, "b");
      if (!scalar_bcast(b)) std::swap(a, b);
      if (scalar_bcast(b) && T_[a].numel == T_[t].numel && T_[a].dt == F32) {
        q.gmul = fld(src(b), "a");
        ops.insert({mo, src(b)});
        t = a;
      }
    }
    const int dv = src(t);
    if (is(dv, "div") && scalar_bcast(fld(dv, "b")) && T_[fld(dv, "a")].numel == T_[t].numel &&
        T_[fld(dv, "a")].dt == F32) {
      q.gdiv = fld(src(fld(dv, "b")), "a");
      q.div_out = t;
      ops.insert({dv, src(fld(dv, "b"))});
      t = fld(dv, "a");
    }
    q.g = t;
    any = any || q.gmul >= 0 || q.gdiv >= 0;
  }
  auto reset = [&]() {
    for (OptParam& q : opt_params_) { q.g = q.final_g; q.gdiv = q.gmul = q.div_out = -1; }
    norm_sums_.clear();
    norm_sum_val_.clear();
    norm_val_.clear();
    norm_prog_[0].clear();
    norm_prog_[1].clear();
    norm_nvals_ = norm_launches_ = 0;
  };
  if (!any) { reset(); return; }
  std::map<int, int> base_of, norm_of;   // gradient tensor -> param index; normalised tensor -> param index
  for (size_t j = 0; j < opt_params_.size(); ++j) {
    base_of[opt_params_[j].g] = (int)j;
    if (opt_params_[j].div_out >= 0) norm_of[opt_params_[j].div_out] = (int)j;
  }
  std::map<int, int> launch_of;   // scalar tensor -> launch index
  bool fail = false;
  std::function<int(int)> visit = [&](int t) -> int {
    auto it = launch_of.find(t);
    if (it != launch_of.end()) return it->second;
    const int op = src(t);
    if (fail || op < 0 || T_[t].numel != 1 || T_[t].dt != F32) { fail = true; return 0; }
    const std::string& k = kinds_[op];
    tgk::ScalarInstr in{tgk::SI_CONST, -1, -1, -1, 0.0};
    int L = 0;
    if (k == "const_scalar") {
      in.k = O(op).at("value").num();
    } else if (k == "sum_last") {
      ops.insert(op);
      int y = fld(op, "a");
      while (is(src(y), "reshape")) { ops.insert(src(y)); y = fld(src(y), "a"); }
      const int mop = src(y);
      if (!is(mop, "mul") || fld(mop, "a") != fld(mop, "b")) { fail = true; return 0; }
      ops.insert(mop);
      const int x = fld(mop, "a");
      NormSum ns{-1, -1, 0};
      if (base_of.count(x)) {
        ns.g = x;
      } else if (norm_of.count(x)) {
        const OptParam& q = opt_params_[norm_of[x]];
        if (visit(q.gdiv) != 0) { fail = true; return 0; }
        ns = {q.g, q.gdiv, 1};
      } else {
        fail = true;
        return 0;
      }
      if (T_[fld(op, "a")].numel != T_[x].numel || T_[x].numel <= 0) { fail = true; return 0; }
      norm_sums_.push_back(ns);
      norm_sum_val_.push_back(norm_nvals_);
      norm_val_[t] = norm_nvals_++;
      return launch_of[t] = ns.launch;
    } else if (k == "add" || k == "sub" || k == "mul" || k == "div" || k == "min" || k == "max") {
      const int la = visit(fld(op, "a")), lb = visit(fld(op, "b"));
      if (fail) return 0;
      in.op = k == "add" ? tgk::SI_ADD : k == "sub" ? tgk::SI_SUB : k == "mul" ? tgk::SI_MUL
             : k == "div" ? tgk::SI_DIV : k == "min" ? tgk::SI_MIN : tgk::SI_MAX;
      in.a = norm_val_.at(fld(op, "a"));
      in.b = norm_val_.at(fld(op, "b"));
      L = std::max(la, lb);
    } else if (k == "add_scalar" || k == "mul_scalar" || k == "sqrt") {
      L = visit(fld(op, "a"));
      if (fail) return 0;
      in.op = k == "add_scalar" ? tgk::SI_ADDK : k == "mul_scalar" ? tgk::SI_MULK : tgk::SI_SQRT;
      in.a = norm_val_.at(fld(op, "a"));
      if (k != "sqrt") in.k = O(op).at("scalar").num();
    } else {
      fail = true;
      return 0;
    }
    ops.insert(op);
    in.out = norm_val_[t] = norm_nvals_++;
    norm_prog_[L].push_back(in);
    return launch_of[t] = L;
  };
  for (const OptParam& q : opt_params_)
    if (q.gdiv >= 0 && visit(q.gdiv) != 0) fail = true;
  for (const OptParam& q : opt_params_)
    if (q.gmul >= 0) visit(q.gmul);
  // A constant another op also reads stays in the graph; the program has its own copy.
  for (auto it = ops.begin(); it != ops.end();) {
    bool outside = false;
    if (kinds_[*it] == "const_scalar")
      for (int c : consumers_[O(*it).at("out").i32()]) if (!ops.count(c) && !adam_ops_.count(c)) outside = true;
    it = outside ? ops.erase(it) : std::next(it);
  }
  norm_launches_ = 1;
  for (const NormSum& s : norm_sums_) norm_launches_ = std::max(norm_launches_, s.launch + 1);
  std::vector<int64_t> elems(norm_launches_, 0);
  for (const NormSum& s : norm_sums_) elems[s.launch] += T_[s.g].numel;
  for (int64_t e : elems) if (e <= 0) fail = true;
  for (const OptParam& q : opt_params_)
    if (!view_[q.g].contiguous() || T_[q.g].numel != T_[q.p].numel || T_[root(q.g)].numel < T_[q.g].numel)
      fail = true;
  if (fail || norm_nvals_ > tgk::kNormMaxVals || !opt_closed(ops, {})) { reset(); return; }
  adam_ops_.insert(ops.begin(), ops.end());
}

// A device copy of a launch table, made once per key: a node bound again (the
// scratch-only launch list) gets the same copy, so rebinding allocates nothing.
const void* Runtime::dev_table(const std::string& key, const void* data, size_t bytes) {
  auto it = table_cache_.find(key);
  if (it != table_cache_.end()) {
    if (it->second.second != bytes) throw Error(TG_INTERNAL, "launch table " + key + " changed size");
    return it->second.first;
  }
  void* dev = nullptr;
  hip_check(hipMalloc(&dev, std::max<size_t>(bytes, 16)), "hipMalloc(table)");
  if (bytes) hip_check(hipMemcpy(dev, data, bytes, hipMemcpyHostToDevice), "hipMemcpy(table)");
  dev_tables_.push_back(dev);
  table_cache_[key] = {dev, bytes};
  return dev;
}

// The fused optimizer's launches, last in the step: the grad_norms launches (value array
// at the start of the workspace, chunk partials after it), then the update.
void Runtime::emit_optimizer() {
  if (opt_params_.empty()) return;
  const size_t vals_bytes = ((size_t)norm_nvals_ * 4 + 255) & ~(size_t)255;
  const int last_op = *adam_ops_.rbegin();
  const int nv = norm_nvals_;
  for (int L = 0; L < norm_launches_; ++L) {
    Node n;
    n.kind = "grad_norm";
    n.op = last_op;
    std::vector<tgk::SqChunk> chunks;
    std::vector<std::pair<int, int64_t>> at;   // chunk -> (gradient tensor, element offset)
    std::vector<int> first, sval;
    double elems = 0;
    for (size_t s = 0; s < norm_sums_.size(); ++s) {
      const NormSum& ns = norm_sums_[s];
      if (ns.launch != L) continue;
      const int slot = (int)first.size();
      first.push_back((int)chunks.size());
      sval.push_back(norm_sum_val_[s]);
      const int64_t N = T_[ns.g].numel;
      const int pre = ns.pre_t >= 0 ? norm_val_.at(ns.pre_t) : -1;
      for (int64_t o = 0; o < N; o += tgk::kNormChunk) {
        chunks.push_back({nullptr, std::min(tgk::kNormChunk, N - o), pre, slot});
        at.emplace_back(ns.g, o);
      }
      n.reads.push_back(root(ns.g));
      elems += (double)N;
    }
    first.push_back((int)chunks.size());
    if (chunks.size() > 0x7fffffffu) throw Error(TG_INVALID_ARGUMENT, "grad_norms: too many gradient chunks");
    n.bytes = 4.0 * elems;
    n.shape = std::to_string(sval.size()) + " sums of squares, " + std::to_string((long long)elems) + " elements";
    n.detail = "mul,sum_last";
    for (const tgk::ScalarInstr& in : norm_prog_[L]) {
      static const char* nm[] = {"const_scalar", "add", "sub", "mul", "div", "min", "max", "add_scalar", "mul_scalar",
                                 "sqrt"};
      n.detail += std::string(",") + nm[in.op];
    }
    n.ws = true;
    const int64_t cb = take_counters((int64_t)sval.size() + 1);
    workspace_bytes_ = std::max(workspace_bytes_, vals_bytes + chunks.size() * sizeof(double));
    const std::vector<tgk::ScalarInstr> prog = norm_prog_[L];
    const std::string key = "norm" + std::to_string(L);
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      std::vector<tgk::SqChunk> ch = chunks;
      for (size_t c = 0; c < ch.size(); ++c) ch[c].g = (const float*)dptr(at[c].first) + at[c].second;
      if (plan_only_) return [](hipStream_t) {};
      tgk::NormLaunch a{};
      a.chunks = (const tgk::SqChunk*)dev_table(key + "c", ch.data(), ch.size() * sizeof(tgk::SqChunk));
      a.nchunks = (int64_t)ch.size();
      a.slot_first = (const int*)dev_table(key + "f", first.data(), first.size() * sizeof(int));
      a.slot_val = (const int*)dev_table(key + "v", sval.data(), sval.size() * sizeof(int));
      a.nslots = (int)sval.size();
      a.prog = prog.empty() ? nullptr
                            : (const tgk::ScalarInstr*)dev_table(key + "p", prog.data(),
                                                                 prog.size() * sizeof(tgk::ScalarInstr));
      a.nprog = (int)prog.size();
      a.vals = cur_ws_;
      a.nvals = nv;
      a.part = reinterpret_cast<double*>(reinterpret_cast<char*>(cur_ws_) + vals_bytes);
      a.counters = cur_counters_ + cb;
      return [a](hipStream_t st) { tgk::grad_norms(a, st); };
    };
    add_node(std::move(n));
  }

  Node n;
  n.kind = opt_sgd_ ? "sgd_multi" : "adam_multi";
  n.op = last_op;
  double elems = 0;
  bool xf = false;
  std::vector<tgk::AdamChunk> chunks;
  std::vector<std::pair<size_t, int64_t>> at;   // chunk -> (param index, element offset)
  for (size_t j = 0; j < opt_params_.size(); ++j) {
    const OptParam& q = opt_params_[j];
    n.reads.push_back(root(q.g));
    n.reads.push_back(root(q.p));
    n.writes.push_back(root(q.p));
    if (q.m >= 0) { n.reads.push_back(root(q.m)); n.writes.push_back(root(q.m)); }
    if (q.v >= 0) { n.reads.push_back(root(q.v)); n.writes.push_back(root(q.v)); }
    n.reads.push_back(root(q.lr));
    if (q.shrink_t >= 0) n.reads.push_back(root(q.shrink_t));
    const int64_t N = T_[q.p].numel;
    if (T_[q.g].numel != N || (q.m >= 0 && T_[q.m].numel != N) || (q.v >= 0 && T_[q.v].numel != N) ||
        T_[root(q.g)].numel < N)
      throw Error(TG_INVALID_ARGUMENT, "optimizer: p / state / gradient size mismatch");
    if (!view_[q.g].contiguous()) throw Error(TG_INTERNAL, "optimizer: gradient is not contiguous");
    const int gd = q.gdiv >= 0 ? norm_val_.at(q.gdiv) : -1, gm = q.gmul >= 0 ? norm_val_.at(q.gmul) : -1;
    xf = xf || gd >= 0 || gm >= 0;
    for (int64_t o = 0; o < N; o += tgk::kAdamChunk) {
      tgk::AdamChunk c{};
      c.shrink = q.shrink;
      c.mom = q.mom;
      c.n = std::min(tgk::kAdamChunk, N - o);
      c.gdiv = gd;
      c.gmul = gm;
      c.flags = q.flags;
      chunks.push_back(c);
      at.emplace_back(j, o);
    }
    elems += (double)N;
    if (opt_sgd_) n.bytes += (q.flags & 4 ? 20.0 : 12.0) * (double)N;
  }
  if (!opt_sgd_) n.bytes = 28.0 * elems;
  n.shape = std::to_string(opt_params_.size()) + " tensors, " + std::to_string((long long)elems) + " params";
  if (xf) n.detail = "div/mul,update";
  n.ws = xf;
  const tgk::AdamHyper h = opt_hyper_;
  const bool sgd = opt_sgd_;
  n.bind = [=]() -> std::function<void(hipStream_t)> {
    std::vector<tgk::AdamChunk> ch = chunks;
    for (size_t c = 0; c < ch.size(); ++c) {
      const OptParam& q = opt_params_[at[c].first];
      const int64_t o = at[c].second;
      ch[c].p = (float*)dptr(q.p) + o;
      ch[c].m = q.m >= 0 ? (float*)dptr(q.m) + o : nullptr;
      ch[c].v = q.v >= 0 ? (float*)dptr(q.v) + o : nullptr;
      ch[c].g = (const float*)dptr(q.g) + o;
      ch[c].shrink_ptr = q.shrink_t >= 0 ? (const float*)dptr(q.shrink_t) : nullptr;
    }
    if (plan_only_) return [](hipStream_t) {};
    const tgk::AdamChunk* dc = (const tgk::AdamChunk*)dev_table("opt", ch.data(), ch.size() * sizeof(tgk::AdamChunk));
    const int64_t nch = (int64_t)ch.size();
    const float* lr = (const float*)dptr(opt_params_.front().lr);
    const float* vals = xf ? cur_ws_ : nullptr;
    if (sgd) return [=](hipStream_t st) { tgk::sgd_multi(dc, nch, lr, vals, st); };
    return [=](hipStream_t st) { tgk::adam_multi(dc, nch, lr, h, vals, st); };
  };
  add_node(std::move(n));
}

void Runtime::lower() {
  if (const char* g = std::getenv("TG_OPT_FUSED")) use_fused_transforms_ = std::string(g) != "0";
  match_optimizer();
  gemm_done_.assign(ops_.size(), 0);
  pool_absorbed_.assign(ops_.size(), 0);
  plan_gemm_groups();
  match_concat_products();
  match_attention();
  match_attention_bwd();
  match_colsums();
  match_gemm_sums();
  defer_colsum_.assign(ops_.size(), 0);
  if (use_gemm_group_)
    for (auto& c : colsum_)
      if (only_optimizer_reads(O(c.first).at("out").i32())) defer_colsum_[c.first] = any_deferred_colsum_ = 1;
  form_groups();
  merge_groups();
  if (use_remat_) remat_groups();
  group_done_.assign(groups_.size(), 0);
  for (size_t i = 0; i < ops_.size(); ++i) {
    if (is_leaf((int)i) || virtual_[i] || cat_absorbed_[i] || pool_absorbed_[i]) continue;
    if (adam_ops_.count((int)i)) continue;
    if (attn_of_[i] >= 0) {
      const int m = attn_of_[i];
      if (m < (int)attn_.size()) {
        if (attn_[m].qk == (int)i) lower_attention(m);
      } else if (attn_bwd_[m - attn_.size()].first == (int)i) {
        lower_attention_bwd(m - (int)attn_.size());
      }
      continue;
    }
    if (mul_absorbed_[i]) continue;
    if (sum_absorbed_[i]) {
      if (gemm_sums_.count((int)i)) lower_gemm_sum((int)i);
      continue;
    }
    if (colsum_.count((int)i)) {
      if (!colsum_done_[i] && !defer_colsum_[i]) lower_colsums((int)i);
      continue;
    }
    int gi = group_of_[i];
    if (gi >= 0) {
      if (groups_[gi].first == (int)i && !group_done_[gi]) {
        DeferredRowSum d{};
        if (use_gemm_group_ && use_colsum_loss_ && (int)deferred_rowsum_.size() < 4 && tail_rowsum(gi, d)) {
          deferred_rowsum_.push_back(d);
          group_done_[gi] = 1;
        } else {
          lower_group(gi);
        }
      }
      continue;
    }
    if (gemm_done_[i]) continue;
    lower_op((int)i);
  }
  flush_deferred_gemms();
  {
    std::vector<int> batch;
    bool scatter_left = !deferred_scatter_.empty(), rows_left = !deferred_rowsum_.empty();
    bool mids_left = !deferred_midsum_.empty();
    const int room = tgk::kColSumMax - (int)deferred_rowsum_.size();   // the first batch takes the row sums
    for (auto& c : colsum_) {
      if (!defer_colsum_[c.first] || colsum_done_[c.first]) continue;
      batch.push_back(c.first);
      if ((int)batch.size() == (rows_left ? room : tgk::kColSumMax)) {
        emit_colsums(batch, scatter_left, rows_left, mids_left);
        scatter_left = rows_left = mids_left = false;
        batch.clear();
      }
    }
    if (!batch.empty()) {
      emit_colsums(batch, scatter_left, rows_left, mids_left);
      scatter_left = rows_left = mids_left = false;
    }
    if (mids_left) throw Error(TG_INTERNAL, "[B, C, L] sums deferred without a column-sum launch");
    if (scatter_left) emit_scatter(deferred_scatter_.front());   // no column sums to join
    if (rows_left)
      for (const DeferredRowSum& d : deferred_rowsum_) lower_group(d.gi);
    deferred_scatter_.clear();
    deferred_rowsum_.clear();
    deferred_midsum_.clear();
  }

  // Drop nodes whose results nobody reads (e.g. a one_hot consumed only by the
  // gather / scatter patterns, which read its indices instead).
  std::set<int> keep;
  for (int o : outputs_) keep.insert(root(o));
  for (auto& c : captures_) keep.insert(root(c.second));
  for (auto& w : copy_writebacks_) keep.insert(root(w.first));
  for (bool changed = true; changed;) {
    changed = false;
    std::set<int> read;
    for (auto& n : nodes_) read.insert(n.reads.begin(), n.reads.end());
    for (const OptParam& q : opt_params_) {
      read.insert(root(q.g));
      read.insert(root(q.lr));
      if (q.shrink_t >= 0) read.insert(root(q.shrink_t));
    }
    for (size_t q = 0; q < nodes_.size(); ++q) {
      bool needed = false;
      for (int w : nodes_[q].writes) if (read.count(w) || keep.count(w)) needed = true;
      if (!needed) { nodes_.erase(nodes_.begin() + q); changed = true; break; }
    }
  }

  emit_optimizer();
}

static std::string shape_str(const Dims& d) {
  std::string s = "[";
  for (size_t i = 0; i < d.size(); ++i) s += (i ? "," : "") + std::to_string(d[i]);
  return s + "]";
}

static const std::map<std::string, int>& pointwise_ops() {
  static const std::map<std::string, int> m = {
      {"add", tgk::FO_ADD}, {"sub", tgk::FO_SUB}, {"mul", tgk::FO_MUL}, {"div", tgk::FO_DIV},
      {"min", tgk::FO_MIN}, {"max", tgk::FO_MAX}, {"less", tgk::FO_LESS}, {"greater", tgk::FO_GREATER},
      {"mul_scalar", tgk::FO_MULS}, {"add_scalar", tgk::FO_ADDS}, {"sqrt", tgk::FO_SQRT}, {"rsqrt", tgk::FO_RSQRT},
      {"log", tgk::FO_LOG}, {"exp", tgk::FO_EXP}, {"relu", tgk::FO_RELU}, {"neg", tgk::FO_NEG},
      {"abs", tgk::FO_ABS}, {"tanh", tgk::FO_TANH}, {"sigmoid", tgk::FO_SIGMOID}, {"erf", tgk::FO_ERF},
      {"sin", tgk::FO_SIN}, {"cos", tgk::FO_COS}, {"relu_grad", tgk::FO_RELU_GRAD}, {"where", tgk::FO_WHERE},
      {"dropout", tgk::FO_DROPOUT}, {"broadcast_to", tgk::FO_COPY}};
  return m;
}

constexpr int64_t kWideRow = 4096;

static bool is_row_reduce_kind(const std::string& k) { return k == "sum_last" || k == "mean_last"; }

// Row shapes of a full shape F = [.., D]: F without its last dim, or with it set to 1.
static int row_class(const Dims& s, const Dims& F) {
  if (F.empty()) return 0;
  Dims a(F.begin(), F.end() - 1);
  if (s == a) return 1;
  a.push_back(1);
  if (s == a) return 2;
  return 0;
}

// Ops that need whole rows (row groups only): last-axis sums (sum_last, mean_last, a
// sum_to_shape that only collapses the last axis) and the row softmaxes.
bool Runtime::is_row_reduce(int m) const {
  const std::string& k = kinds_[m];
  if (is_row_reduce_kind(k)) return true;
  if (k == "log_softmax_last") return true;
  if (k == "softmax_causal_last") {
    const Dims& in = T_[fld(m, "a")].shape;
    return in.size() >= 2 && in[in.size() - 2] == in.back();
  }
  if (k != "sum_to_shape") return false;
  const Dims& in = T_[fld(m, "a")].shape;
  const Dims& out = T_[O(m).at("out").i32()].shape;
  return !in.empty() && in.back() > 1 && row_class(out, in) == 2;
}

// The group whose member produced tensor t's values, when t is that member's output or
// a contiguous full-size view of it (a reshape keeps the flat order); -1 otherwise.
int Runtime::producer_group(int t) const {
  const int r = root(t);
  const int src = T_[r].src;
  if (src < 0 || group_of_[src] < 0) return -1;
  if (t != r && !(view_[t].contiguous() && T_[t].numel == T_[r].numel)) return -1;
  if (O(src).at("out").i32() != r) return -1;
  return group_of_[src];
}

// Broadcast class of member m's operands: 0 = full (element groups, reductions and
// full-shaped members of row groups), 1 / 2 = row-shaped member ([..] / [.., 1]).
int Runtime::op_class(int m, bool row, const Dims& F) const {
  if (!row || is_row_reduce(m)) return 0;
  if (kinds_[m] == "one_hot") return 1;   // its indices are one value per row
  return row_class(T_[O(m).at("out").i32()].shape, F);
}

// The one_hot op whose result operand t of a row group of shape F = [.., D] is, when the
// group can evaluate it in registers instead of reading it: t is the whole result, of
// shape F with depth D, and its i32 indices (shape F without D) are a graph input, so they
// exist before any group runs. -1 otherwise.
int Runtime::inline_one_hot(int t, const Dims& F) const {
  const int r = root(t);
  const int s = T_[r].src;
  if (s < 0 || kinds_[s] != "one_hot" || virtual_[s] || F.empty() || T_[t].shape != F) return -1;
  if (t != r && !(view_[t].contiguous() && T_[t].numel == T_[r].numel)) return -1;
  if (O(s).at("out").i32() != r || O(s).at("depth").i64() != F.back()) return -1;
  const int ix = fld(s, "indices");
  const int ixs = T_[root(ix)].src;
  if (T_[ix].dt != I32 || T_[ix].shape != Dims(F.begin(), F.end() - 1)) return -1;
  if (ixs >= 0 && !is_leaf(ixs)) return -1;
  return s;
}

bool Runtime::dup_in(int gi, int m) const {
  const std::vector<int>& d = groups_[gi].dups;
  return std::find(d.begin(), d.end(), m) != d.end();
}

Runtime::GroupPlan Runtime::plan_group(const std::vector<int>& own, bool row, const Dims& F,
                                       const std::vector<int>* dups) const {
  const auto& pw = pointwise_ops();
  GroupPlan gp;
  // members in graph order (a topological order): the group's own ops and its recomputed ones
  std::vector<int> ops(own);
  const std::set<int> dup(dups ? dups->begin() : own.end(), dups ? dups->end() : own.end());
  ops.insert(ops.end(), dup.begin(), dup.end());
  // A row group evaluates its one-hot operands from their indices (a compare with the
  // column) as members of its own that store nothing.
  std::set<int> inl;
  if (row)
    for (int m : ops)
      for (int t : op_inputs(*ops_[m])) {
        const int s = inline_one_hot(t, F);
        if (s >= 0) inl.insert(s);
      }
  ops.insert(ops.end(), inl.begin(), inl.end());
  std::sort(ops.begin(), ops.end());
  std::set<int> members(ops.begin(), ops.end());
  auto inside = [&](int t) {
    if (row && inline_one_hot(t, F) >= 0) return true;
    const int gi = producer_group(t);
    return gi >= 0 && members.count(T_[root(t)].src) > 0;
  };
  // operands per member, in instruction order
  std::vector<std::vector<int>> opnds(ops.size());
  for (size_t q = 0; q < ops.size(); ++q) {
    const int m = ops[q];
    const std::string& k = kinds_[m];
    const tgj::Value& op = O(m);
    if (k == "relu_grad") opnds[q] = {op.at("x").i32(), op.at("dy").i32()};
    else if (k == "one_hot") opnds[q] = {op.at("indices").i32()};
    else if (k == "where") opnds[q] = {op.at("cond").i32(), op.at("a").i32(), op.at("b").i32()};
    else if (op.get("b") && k != "dropout") opnds[q] = {op.at("a").i32(), op.at("b").i32()};
    else opnds[q] = {op.at("a").i32()};
    if (k == "dropout") gp.seed = op.at("seed").i32();
  }
  // external operands
  for (size_t q = 0; q < ops.size(); ++q) {
    const int cls = op_class(ops[q], row, F);
    for (int t : opnds[q]) {
      if (inside(t)) continue;
      std::pair<int, int> key{t, cls};
      if (std::find(gp.ext.begin(), gp.ext.end(), key) == gp.ext.end()) gp.ext.push_back(key);
    }
  }
  // stored outputs: members read outside the group, graph outputs, captures, writeback sources
  std::set<int> must_store;
  for (int o : outputs_) must_store.insert(o);
  for (auto& c : captures_) must_store.insert(c.second);
  for (auto& w : copy_writebacks_) must_store.insert(w.first);
  // A contiguous full-size view (reshape) of a member's output that only members read is
  // read from the register, not from memory.
  std::function<bool(int)> read_outside = [&](int t) -> bool {
    if (must_store.count(t)) return true;
    for (int c : consumers_[t]) {
      if (members.count(c)) continue;
      // a group that evaluates t's producer again reads nothing of t (nor do the
      // recomputed copies of a dropped consumer: their groups recompute t's producer too)
      if (group_of_[c] >= 0 && (dup_in(group_of_[c], T_[root(t)].src) || dropped_[c])) continue;
      if (virtual_[c]) {
        const int v = O(c).at("out").i32();
        if (root(v) == root(t) && view_[v].contiguous() && T_[v].numel == T_[root(v)].numel && !read_outside(v))
          continue;
      }
      return true;
    }
    return false;
  };
  std::vector<bool> stored(ops.size(), false);
  for (size_t q = 0; q < ops.size(); ++q) {
    if (dup.count(ops[q]) || inl.count(ops[q])) continue;   // the owning group stores what others read
    const int t = O(ops[q]).at("out").i32();
    if (read_outside(t)) { stored[q] = true; gp.outs.push_back(t); }
  }
  // last read of every value (ext operand index or member position)
  std::map<int, int> member_pos;   // producing op -> position
  for (size_t q = 0; q < ops.size(); ++q) member_pos[ops[q]] = (int)q;
  std::vector<int> ext_last(gp.ext.size(), -1), val_last(ops.size(), -1);
  auto ref = [&](size_t q, int t, int cls) -> std::pair<bool, int> {   // (is_member, index)
    if (inside(t)) return {true, member_pos.at(T_[root(t)].src)};
    const auto it = std::find(gp.ext.begin(), gp.ext.end(), std::make_pair(t, cls));
    return {false, (int)(it - gp.ext.begin())};
  };
  for (size_t q = 0; q < ops.size(); ++q) {
    const int cls = op_class(ops[q], row, F);
    for (int t : opnds[q]) {
      auto r = ref(q, t, cls);
      if (r.first) val_last[r.second] = (int)q;
      else ext_last[r.second] = (int)q;
    }
  }
  // linear scan: ext operands take registers 0..n_ext-1 before the first instruction
  std::vector<int> ext_reg(gp.ext.size()), val_reg(ops.size(), -1);
  std::vector<bool> busy;
  auto take = [&]() {
    for (size_t r = 0; r < busy.size(); ++r) if (!busy[r]) { busy[r] = true; return (int)r; }
    busy.push_back(true);
    return (int)busy.size() - 1;
  };
  for (size_t e = 0; e < gp.ext.size(); ++e) ext_reg[e] = take();
  for (size_t q = 0; q < ops.size(); ++q) {
    const int m = ops[q];
    const std::string& k = kinds_[m];
    const tgj::Value& op = O(m);
    const int cls = op_class(m, row, F);
    tgk::FusedInstr in{};
    std::vector<int> regs;
    for (int t : opnds[q]) {
      auto r = ref(q, t, cls);
      regs.push_back(r.first ? val_reg[r.second] : ext_reg[r.second]);
    }
    auto DT = [&](int t) { return kdt(T_[t].dt); };
    in.a = regs[0];
    in.ta = DT(opnds[q][0]);
    if (regs.size() > 1) { in.b = regs[1]; in.tb = DT(opnds[q][1]); }
    if (regs.size() > 2) in.c = regs[2];
    const int out = op.at("out").i32();
    in.dt = kdt(T_[out].dt);
    if (k == "one_hot") {
      in.op = tgk::FO_ONEHOT;
    } else if (k == "softmax_causal_last") {
      in.op = tgk::FO_SOFTMAX_CAUSAL;
    } else if (k == "log_softmax_last") {
      in.op = tgk::FO_LOG_SOFTMAX;
    } else if (is_row_reduce(m)) {
      in.op = tgk::FO_ROWSUM;
      in.imm = k == "mean_last" ? (double)F.back() : 1.0;
    } else {
      in.op = pw.at(k);
      if (k == "mul_scalar" || k == "add_scalar") in.imm = op.at("scalar").num();
      if (k == "dropout") {
        const double p = op.at("p").num();
        in.imm = p;
        in.imm2 = 1.0 / (1.0 - p);
        in.salt = (uint32_t)(uint64_t)std::fmod((double)op.at("salt").i64() * 2654435761.0, 4294967296.0);
      }
      // Inexpensive f32 forms of the arithmetic ops.
      if (in.ta == tgk::DT_F32 && in.tb == tgk::DT_F32 && in.dt == tgk::DT_F32) {
        if (in.op == tgk::FO_ADD) in.op = tgk::FO_FADD;
        else if (in.op == tgk::FO_SUB) in.op = tgk::FO_FSUB;
        else if (in.op == tgk::FO_MUL) in.op = tgk::FO_FMUL;
        else if (in.op == tgk::FO_DIV) in.op = tgk::FO_FDIV;
      }
    }
    // free operands read for the last time here (an instruction reads all operands of an
    // element before writing its result, so dst may reuse one of them)
    for (int t : opnds[q]) {
      auto r = ref(q, t, cls);
      if (r.first) { if (val_last[r.second] == (int)q && !stored[r.second]) busy[val_reg[r.second]] = false; }
      else if (ext_last[r.second] == (int)q) busy[ext_reg[r.second]] = false;
    }
    in.dst = val_reg[q] = take();
    if (val_last[q] < 0 && !stored[q]) busy[in.dst] = false;   // dead value
    gp.code.push_back(in);
  }
  for (size_t q = 0; q < ops.size(); ++q)
    if (stored[q]) gp.out_reg.push_back(val_reg[q]);
  gp.nregs = (int)busy.size();
  return gp;
}

// Greedy convex grouping. An op joins a group that produces one of its inputs if every
// operand is produced inside the group or available before the group's first op (an
// earlier op, a leaf, or an earlier group), so the whole group can run at its first op's
// position without reordering anything else. Same-shape pointwise ops form element
// groups; a last-axis sum / mean turns its group into a row group, which may also hold
// pointwise ops on the row shape (LayerNorm, softmax and cross-entropy chains).
void Runtime::form_groups() {
  group_of_.assign(ops_.size(), -1);
  dropped_.assign(ops_.size(), 0);
  groups_.clear();
  const auto& pw = pointwise_ops();
  // Position at which a tensor's data exists (views resolve to their root).
  auto eff_pos = [&](int t) {
    int r = root(t);
    int src = T_[r].src;
    if (src < 0 || is_leaf(src)) return -1;
    return group_of_[src] >= 0 ? groups_[group_of_[src]].first : src;
  };
  auto fits = [&](const std::vector<int>& ops, bool row, const Dims& F) {
    if (ops.size() > (size_t)tgk::kFusedMaxInstr) return false;
    GroupPlan gp = plan_group(ops, row, F);
    // a wide row keeps 64 or more values per lane in each register: few registers
    const int maxregs = row && F.back() > 1024 ? 4 : tgk::kFusedRegs;
    return gp.ext.size() <= (size_t)tgk::kFusedMaxIn && gp.outs.size() <= (size_t)tgk::kFusedMaxOut &&
           gp.nregs <= maxregs;
  };
  for (size_t i = 0; i < ops_.size(); ++i) {
    const std::string& k = kinds_[i];
    if (virtual_[i] || is_leaf((int)i) || attn_of_[i] >= 0 || mul_absorbed_[i] || sum_absorbed_[i] ||
        colsum_.count((int)i) || adam_ops_.count((int)i))
      continue;
    const bool red = is_row_reduce((int)i);
    if (!red && !pw.count(k)) continue;
    const int out = ops_[i]->at("out").i32();
    const Dims& So = T_[out].shape;
    if (T_[out].numel <= 0) continue;
    Dims In;
    if (red) {
      const int a = fld((int)i, "a");
      In = T_[a].shape;
      // Rows up to 1024 wide; a single row (a whole-tensor sum) up to kWideRow in generated
      // kernels. Wider rows run as standalone reductions.
      const int64_t maxd = use_jit_ && T_[a].numel == In.back() ? kWideRow : 1024;
      if (In.empty() || In.back() < 1 || In.back() > maxd || T_[a].numel <= 0) continue;
    }
    std::vector<int> cands;
    for (int t : op_inputs(*ops_[i])) {
      const int gi = producer_group(t);
      if (gi >= 0 && std::find(cands.begin(), cands.end(), gi) == cands.end()) cands.push_back(gi);
      // a recent group that already reads t (a sibling): joining it needs every input of
      // op i to exist before that group runs, which the checks below require
      for (int c : consumers_[t]) {
        if (c >= (int)i || group_of_[c] < 0) continue;
        const int sg = group_of_[c];
        if ((int)i - groups_[sg].first > 64) continue;
        if (std::find(cands.begin(), cands.end(), sg) == cands.end()) cands.push_back(sg);
      }
    }
    std::sort(cands.begin(), cands.end(), [&](int a, int b) { return groups_[a].first > groups_[b].first; });
    // Group gi can run at position i instead of at its first op when nothing outside it
    // reads its members' results before i (through views; patterns other than plain ops
    // and groups are not moved around).
    auto movable_to_i = [&](int gi) {
      std::vector<int> stack;
      for (int m : groups_[gi].ops) stack.push_back(ops_[m]->at("out").i32());
      while (!stack.empty()) {
        const int t = stack.back();
        stack.pop_back();
        for (int c : consumers_[t]) {
          if (group_of_[c] == gi || c == (int)i) continue;
          if (virtual_[c] && !is_leaf(c) && kinds_[c] != "matmul" && kinds_[c] != "matmul_batched") {
            stack.push_back(ops_[c]->at("out").i32());
            continue;
          }
          if (attn_of_[c] >= 0 || mul_absorbed_[c] || sum_absorbed_[c] || colsum_.count(c)) return false;
          const int pos = group_of_[c] >= 0 ? groups_[group_of_[c]].first : c;
          if (pos <= (int)i) return false;
        }
      }
      return true;
    };
    int joined = -1;
    for (int gi : cands) {
      Group& g = groups_[gi];
      const Dims& F = g.shape;
      bool ok = true;
      bool late = false;   // an input of op i exists only after the group's first op
      bool becomes_row = g.row;
      if (red) {
        ok = T_[fld((int)i, "a")].shape == F;
        becomes_row = true;
      } else if (!g.row) {
        ok = So == F;
      } else {
        const int cls = row_class(So, F);
        ok = So == F || (cls > 0 && k != "dropout");
      }
      for (int t : op_inputs(*ops_[i])) {
        if (!ok) break;
        const bool in_g = producer_group(t) == gi;
        if (!in_g) {
          if (eff_pos(t) >= g.first) late = true;
          continue;
        }
        if (k == "dropout" && t == fld((int)i, "seed")) continue;
        const Dims& ts = T_[t].shape;
        if (red) continue;   // the reduced input has shape F (checked above)
        if (!g.row) { if (ts != F) ok = false; continue; }
        if (So == F) { if (!(ts == F || row_class(ts, F) == 2)) ok = false; }
        else if (ts != So) ok = false;
      }
      if (ok && late) ok = movable_to_i(gi);
      if (!ok) continue;
      std::vector<int> ops = g.ops;
      ops.push_back((int)i);
      if (!fits(ops, becomes_row, F)) continue;
      g.ops.push_back((int)i);
      g.row = becomes_row;
      if (late) g.first = (int)i;   // the group now runs where its last input exists
      group_of_[i] = gi;
      joined = gi;
      break;
    }
    if (joined < 0) {
      Group g{(int)i, {(int)i}, red ? In : So, red};
      if (!fits(g.ops, g.row, g.shape)) continue;
      groups_.push_back(g);
      group_of_[i] = (int)groups_.size() - 1;
    }
  }
}

// A group B runs inside an earlier group A of the same shape when B reads a result of A
// and every other tensor B reads exists where A runs (a leaf, or a result produced before
// A's first op): one launch instead of two, and values of A that only B read stay in
// registers. Members keep their per-element code, so the results are the same bits. (The
// cross-entropy gradient rows start from a constant broadcast, so form_groups finds no
// input tying them to the log-softmax rows they read.)
void Runtime::merge_groups() {
  auto eff_pos = [&](int t) {
    const int r = root(t);
    const int src = T_[r].src;
    if (src < 0 || is_leaf(src)) return -1;
    return group_of_[src] >= 0 ? groups_[group_of_[src]].first : src;
  };
  // Ops whose node runs once at runtime creation (split_init_nodes: it reads only such
  // results and writes nothing pinned): constants, and groups of constant arithmetic.
  std::set<int> pinned;
  for (int o : outputs_) pinned.insert(root(o));
  for (auto& c : captures_) pinned.insert(root(c.second));
  for (auto& w : copy_writebacks_) pinned.insert(root(w.first));
  std::vector<signed char> memo(ops_.size(), -1);
  std::function<bool(int)> init_op = [&](int m) -> bool {
    if (memo[m] >= 0) return memo[m] != 0;
    memo[m] = 0;
    bool r = false;
    const std::string& k = kinds_[m];
    if (k == "const_scalar" || k == "const_fill" || k == "arange") {
      r = !pinned.count(root(O(m).at("out").i32()));
    } else if (group_of_[m] >= 0) {
      const int g = group_of_[m];
      r = true;
      for (int q : groups_[g].ops) {
        if (pinned.count(root(O(q).at("out").i32()))) r = false;
        for (int t : op_inputs(*ops_[q])) {
          const int src = T_[root(t)].src;
          if (src >= 0 && group_of_[src] == g) continue;
          if (src < 0 || is_leaf(src) || !init_op(src)) r = false;
        }
      }
    }
    memo[m] = r ? 1 : 0;
    return r;
  };
  std::vector<char> init_group(groups_.size(), 0);
  for (size_t g = 0; g < groups_.size(); ++g)
    if (!groups_[g].ops.empty()) init_group[g] = init_op(groups_[g].ops.front());
  for (size_t b = 0; b < groups_.size(); ++b) {
    if (init_group[b]) continue;
    for (size_t a = 0; a < groups_.size() && !groups_[b].ops.empty(); ++a) {
      const Group& A = groups_[a];
      const Group& B = groups_[b];
      if (a == b || init_group[a] || A.ops.empty() || A.first >= B.first || A.shape != B.shape) continue;
      const Dims& F = A.shape;
      const bool row = A.row || B.row;
      bool ok = true, reads_a = false;
      for (int m : B.ops) {
        const int so = O(m).at("out").i32();
        const Dims& So = T_[so].shape;
        for (int t : op_inputs(*ops_[m])) {
          const int pg = producer_group(t);
          if (pg != (int)a && pg != (int)b) {
            const int src = T_[root(t)].src;
            if (src >= 0 && !is_leaf(src) && init_op(src)) continue;   // exists before any step launch
            if (eff_pos(t) >= A.first) ok = false;
            continue;
          }
          if (pg == (int)a) reads_a = true;
          // the operand shapes a member may read from its own group (form_groups' rule)
          if (kinds_[m] == "dropout" && t == fld(m, "seed")) continue;
          if (is_row_reduce(m)) continue;
          const Dims& ts = T_[t].shape;
          if (!row) ok = ok && ts == F;
          else if (So == F) ok = ok && (ts == F || row_class(ts, F) == 2);
          else ok = ok && ts == So;
        }
        if (!ok) break;
      }
      if (!ok || !reads_a) continue;
      std::vector<int> ops = A.ops;
      ops.insert(ops.end(), B.ops.begin(), B.ops.end());
      std::sort(ops.begin(), ops.end());
      if (ops.size() > (size_t)tgk::kFusedMaxInstr) continue;
      const GroupPlan gp = plan_group(ops, row, F);
      const int maxregs = row && F.back() > 1024 ? 4 : tgk::kFusedRegs;
      if (gp.ext.size() > (size_t)tgk::kFusedMaxIn || gp.outs.size() > (size_t)tgk::kFusedMaxOut || gp.nregs > maxregs)
        continue;
      for (int m : groups_[b].ops) group_of_[m] = (int)a;
      groups_[a].ops = ops;
      groups_[a].row = row;
      groups_[b].ops.clear();
    }
  }
}

// Recomputation instead of storage. An element group G that reads values a pointwise
// chain of another group P produced (same shape as G, no dropout, no row reductions)
// evaluates that chain again from the chain's own inputs, tensors in memory (GEMM
// outputs, parameters, other nodes' results), when that reads fewer full-size tensors
// than it saves. Every reader of a recomputed value must be P or G, so a value all of
// whose outside readers recompute it is no longer stored by P, and P drops members no
// stored value needs. Recomputed ops run the same per-element code, so the values are
// the same bits. (For a GELU layer: the forward group stops storing the erf and exp
// terms of the derivative, the backward group evaluates them from the pre-activation
// GEMM output.)
void Runtime::remat_groups() {
  const auto& pw = pointwise_ops();
  // ops whose f64 evaluation costs more than reading their f32 result back
  static const std::set<std::string> costly = {"erf", "tanh", "sigmoid", "sin", "cos"};
  bool any = false;
  for (size_t gi = 0; gi < groups_.size(); ++gi) {
    Group& G = groups_[gi];
    if (G.row || G.ops.empty()) continue;
    const GroupPlan gp = plan_group(G.ops, false, G.shape, &G.dups);
    const int64_t full = prod(G.shape);
    std::set<int> ext_roots;
    for (auto& e : gp.ext) ext_roots.insert(root(e.first));
    std::set<int> cone, leaves;
    int pulled = 0;
    for (auto& e : gp.ext) {
      const int t = e.first;
      if (e.second != 0 || t != root(t) || T_[t].numel < full) continue;
      const int P = producer_group(t);
      if (P < 0 || P == (int)gi) continue;
      std::set<int> c2 = cone, l2 = leaves;
      bool ok = true;
      std::function<void(int)> visit = [&](int u) {
        if (!ok) return;
        const int pg = producer_group(u);
        if (pg < 0) { l2.insert(u); return; }
        const int m = T_[root(u)].src;
        if (c2.count(m)) return;
        if (u != root(u) || !pw.count(kinds_[m]) || kinds_[m] == "dropout" || T_[u].shape != G.shape ||
            costly.count(kinds_[m])) {
          ok = false;
          return;
        }
        for (int c : consumers_[u])
          if (group_of_[c] != pg && group_of_[c] != (int)gi) { ok = false; return; }
        c2.insert(m);
        for (int v : op_inputs(*ops_[m])) visit(v);
      };
      visit(t);
      if (!ok) continue;
      cone = std::move(c2);
      leaves = std::move(l2);
      ++pulled;
    }
    if (pulled == 0) continue;
    int new_reads = 0;
    for (int l : leaves)
      if (!ext_roots.count(root(l)) && T_[l].numel >= full) ++new_reads;
    if (new_reads >= pulled) continue;
    std::vector<int> dups = G.dups;
    for (int m : cone) dups.push_back(m);
    const GroupPlan np = plan_group(G.ops, false, G.shape, &dups);
    if (np.ext.size() > (size_t)tgk::kFusedMaxIn || np.outs.size() > (size_t)tgk::kFusedMaxOut ||
        np.nregs > tgk::kFusedRegs || np.code.size() > (size_t)tgk::kFusedMaxInstr)
      continue;
    G.dups = dups;
    any = true;
  }
  if (!any) return;
  // drop the members whose results no stored value of their group needs any more
  for (Group& P : groups_) {
    if (P.ops.empty()) continue;
    const GroupPlan gp = plan_group(P.ops, P.row, P.shape, &P.dups);
    std::set<int> mem(P.ops.begin(), P.ops.end());
    mem.insert(P.dups.begin(), P.dups.end());
    std::set<int> live;
    std::vector<int> work;
    for (int m : mem)
      if (std::find(gp.outs.begin(), gp.outs.end(), O(m).at("out").i32()) != gp.outs.end()) {
        live.insert(m);
        work.push_back(m);
      }
    while (!work.empty()) {
      const int m = work.back();
      work.pop_back();
      for (int u : op_inputs(*ops_[m])) {
        const int src = T_[root(u)].src;
        if (src >= 0 && mem.count(src) && live.insert(src).second) work.push_back(src);
      }
    }
    auto dead = [&](int m) { return !live.count(m); };
    for (int m : P.ops)
      if (dead(m)) dropped_[m] = 1;
    P.ops.erase(std::remove_if(P.ops.begin(), P.ops.end(), dead), P.ops.end());
    P.dups.erase(std::remove_if(P.dups.begin(), P.dups.end(), dead), P.dups.end());
  }
}

void Runtime::lower_group(int gi) {
  const Group& g = groups_[gi];
  const Dims F = g.shape;
  const bool row = g.row;
  if (g.ops.empty()) return;   // every result recomputed where it is read
  GroupPlan gp = plan_group(g.ops, row, F, &g.dups);
  if (gp.ext.size() > (size_t)tgk::kFusedMaxIn || gp.outs.size() > (size_t)tgk::kFusedMaxOut ||
      gp.nregs > tgk::kFusedRegs)
    throw Error(TG_INTERNAL, "fused group exceeds the kernel's limits");
  Node n;
  n.op = g.first;
  n.kind = row ? "rowfused" : (g.ops.size() == 1 ? "elementwise" : "fused");
  n.shape = shape_str(F) + " x" + std::to_string(g.ops.size());
  if (!g.dups.empty()) n.shape += " +" + std::to_string(g.dups.size()) + " recomputed";
  for (size_t q = 0; q < g.ops.size(); ++q) n.detail += (q ? "," : "") + kinds_[g.ops[q]];
  for (auto& e : gp.ext) n.reads.push_back(root(e.first));
  if (gp.seed >= 0) n.reads.push_back(root(gp.seed));
  for (int t : gp.outs) n.writes.push_back(root(t));
  double bytes = 0;
  std::set<int> counted;
  for (auto& e : gp.ext) if (counted.insert(e.first).second) bytes += 4.0 * T_[e.first].numel;
  for (int t : gp.outs) bytes += 4.0 * T_[t].numel;
  n.bytes = bytes;
  const size_t code_off = fused_code_.size();
  fused_code_.insert(fused_code_.end(), gp.code.begin(), gp.code.end());
  const int seed = gp.seed;
  const size_t slot = programs_.size();
  programs_.emplace_back();
  n.bind = [=]() -> std::function<void(hipStream_t)> {
    tgk::FusedProgram& p = programs_[slot];
    memset(&p, 0, sizeof(p));
    const int64_t cnt = prod(F);
    if (cnt >= (int64_t(1) << 31)) throw Error(TG_INVALID_ARGUMENT, "fused group: 2^31 or more elements");
    // Broadcast strides of every operand over F (row-class operands broadcast against the
    // row shape, then stride 0 along D).
    const size_t nx = gp.ext.size();
    std::vector<Dims> bs(nx, Dims(F.size(), 0));
    for (size_t q = 0; q < nx; ++q) {
      const int t = gp.ext[q].first, cls = gp.ext[q].second;
      const View& v = view_[t];
      if (T_[v.root].numel >= (int64_t(1) << 31)) throw Error(TG_INVALID_ARGUMENT, "fused group: operand too large");
      const size_t rankS = cls == 1 ? F.size() - 1 : F.size();
      const int off = (int)rankS - (int)v.dims.size();
      if (off < 0) throw Error(TG_INTERNAL, "fused group: operand rank exceeds its consumer's");
      for (size_t d = 0; d < v.dims.size(); ++d) bs[q][off + d] = v.dims[d] == 1 ? 0 : v.strides[d];
      if (cls > 0) bs[q][F.size() - 1] = 0;
      check_span("fused operand", T_[v.root].numel, 0, F.data(), bs[q].data(), (int)F.size());
    }
    // Iteration dims: element groups merge all dims; row groups merge the row dims and keep
    // D apart. Size-1 dims are dropped.
    const size_t nmerge = row ? F.size() - 1 : F.size();
    Dims md;
    std::vector<Dims> ms(nx);
    for (size_t d = 0; d < nmerge; ++d) {
      if (F[d] == 1) continue;
      bool merge = !md.empty();
      for (size_t q = 0; q < nx && merge; ++q) merge = ms[q].back() == bs[q][d] * F[d];
      if (merge) {
        md.back() *= F[d];
        for (size_t q = 0; q < nx; ++q) ms[q].back() = bs[q][d];
      } else {
        md.push_back(F[d]);
        for (size_t q = 0; q < nx; ++q) ms[q].push_back(bs[q][d]);
      }
    }
    auto aligned = [](const void* ptr) { return ((uintptr_t)ptr & 15) == 0; };
    p.n_in = (int)nx;
    p.nregs = gp.nregs;
    if (row) {
      const int64_t D = F.back();
      if (md.empty()) { md.push_back(1); for (auto& m : ms) m.push_back(0); }
      if (md.size() > (size_t)tgk::kMaxRank) throw Error(TG_INTERNAL, "fused group: rank too large");
      p.row_d = (int32_t)D;
      p.vec = 1;
      p.rank = (int)md.size();
      for (int d = 0; d < p.rank; ++d) p.div[d] = tgk::make_fastdiv((uint32_t)md[d]);
      for (size_t q = 0; q < nx; ++q) {
        p.in[q] = ptr_[view_[gp.ext[q].first].root];
        p.in_dt[q] = kdt(T_[gp.ext[q].first].dt);
        p.in_mode[q] = tgk::FM_STRIDED;
        p.in_inner[q] = (int32_t)bs[q][F.size() - 1];
        for (int d = 0; d < p.rank; ++d) p.in_strides[q][d] = (int32_t)ms[q][d];
      }
    } else {
      if (md.empty()) { md.push_back(1); for (auto& m : ms) m.push_back(0); }
      if (md.size() > (size_t)tgk::kMaxRank) throw Error(TG_INTERNAL, "fused group: rank too large");
      const int R = (int)md.size();
      const Dims cs = contiguous_strides(md);
      // Four elements per thread when the innermost dim allows it and every 128-bit access
      // is aligned.
      bool v4 = md[R - 1] % 4 == 0;
      std::vector<int> mode(nx);
      for (size_t q = 0; q < nx; ++q) {
        bool contig = true, scalar = true;
        for (int d = 0; d < R; ++d) {
          if (ms[q][d] != cs[d]) contig = false;
          if (ms[q][d] != 0) scalar = false;
        }
        mode[q] = contig ? tgk::FM_CONTIG : (scalar ? tgk::FM_SCALAR : tgk::FM_STRIDED);
        if (contig && !aligned(ptr_[view_[gp.ext[q].first].root])) v4 = false;
      }
      for (int t : gp.outs) if (!aligned(dptr(t))) v4 = false;
      const int vec = v4 ? 4 : 1;
      p.vec = vec;
      p.rank = R;
      for (int d = 0; d < R; ++d) p.div[d] = tgk::make_fastdiv((uint32_t)(d == R - 1 ? md[d] / vec : md[d]));
      for (size_t q = 0; q < nx; ++q) {
        const View& v = view_[gp.ext[q].first];
        p.in[q] = ptr_[v.root];
        p.in_dt[q] = kdt(T_[gp.ext[q].first].dt);
        int m = mode[q];
        const int64_t inner = ms[q][R - 1];
        if (m == tgk::FM_STRIDED && vec == 4) {
          bool outer4 = aligned(ptr_[v.root]);
          for (int d = 0; d < R - 1; ++d) if (ms[q][d] % 4) outer4 = false;
          if (inner == 1 && outer4) m = tgk::FM_STRIDED_V;
          else if (inner == 0) m = tgk::FM_STRIDED_B;
        }
        p.in_mode[q] = m;
        p.in_inner[q] = (int32_t)inner;
        if (m != tgk::FM_CONTIG && m != tgk::FM_SCALAR) p.any_strided = 1;
        for (int d = 0; d < R; ++d) p.in_strides[q][d] = (int32_t)(d == R - 1 ? inner * vec : ms[q][d]);
      }
    }
    p.n_out = (int)gp.outs.size();
    for (size_t q = 0; q < gp.outs.size(); ++q) {
      const int t = gp.outs[q];
      p.out[q] = dptr(t);
      p.out_dt[q] = kdt(T_[t].dt);
      p.out_reg[q] = gp.out_reg[q];
      const bool rowout = row && row_class(T_[t].shape, F) > 0;
      p.out_row[q] = rowout ? 1 : 0;
      const int64_t need = rowout ? cnt / F.back() : cnt;
      if (T_[root(t)].numel < need || T_[t].numel != need) throw Error(TG_INTERNAL, "fused group: output size mismatch");
    }
    p.seed = seed >= 0 ? (const int32_t*)dptr(seed) : nullptr;
    p.n_instr = (int)gp.code.size();
    p.code = fused_code_dev_ + code_off;
    const int64_t nthreads = row ? cnt / F.back() : cnt / p.vec;
    if (!use_jit_) return [this, slot, nthreads](hipStream_t st) { tgk::fused(programs_[slot], nthreads, st); };
    tgk::JitKernel jk = tgk::fused_kernel(p, fused_code_.data() + code_off, nthreads);
    const size_t js = jit_slots_.size();
    jit_slots_.emplace_back();
    JitSlot& sl = jit_slots_.back();
    sl.name = jk.name;
    sl.grid = jk.grid;
    for (int k = 0; k < p.n_in; ++k) sl.args.in[k] = p.in[k];
    for (int k = 0; k < p.n_out; ++k) sl.args.out[k] = p.out[k];
    sl.args.seed = p.seed;
    jit_pending_.push_back(std::move(jk));
    return [this, js](hipStream_t st) { launch_jit(js, st); };
  };
  add_node(std::move(n));
}


// Attention chains the fused kernel covers: shapes it supports, unit-stride head dims
// and 16-byte aligned rows, intermediate products read by nothing else, and v available
// at the first product (where the fused node runs). TG_ATTN=0 in the environment keeps
// the ops unfused.
void Runtime::match_attention() {
  attn_of_.assign(ops_.size(), -1);
  attn_.clear();
  if (const char* e = std::getenv("TG_ATTN"))
    if (std::string(e) == "0") return;
  auto only = [&](int t) { return consumers_[t].size() == 1 ? consumers_[t][0] : -1; };
  auto pinned = [&](int t) {
    for (int o : outputs_) if (o == t) return true;
    for (auto& c : captures_) if (c.second == t) return true;
    for (auto& w : copy_writebacks_) if (w.first == t) return true;
    return false;
  };
  for (size_t i = 0; i < ops_.size(); ++i) {
    if (kinds_[i] != "matmul_batched" || virtual_[i]) continue;
    AttnMatch m{(int)i, -1, -1, -1, -1};
    const int S = O((int)i).at("out").i32();
    if (pinned(S)) continue;
    int c = only(S), S2 = S;
    if (c >= 0 && kinds_[c] == "mul_scalar" && T_[S].dt == F32) {
      m.scale = c;
      S2 = O(c).at("out").i32();
      if (pinned(S2)) continue;
      c = only(S2);
    }
    if (c < 0 || kinds_[c] != "softmax_causal_last" || fld(c, "a") != S2) continue;
    m.softmax = c;
    const int P = O(c).at("out").i32();
    int Pd = P;
    for (int u : consumers_[P])
      if (kinds_[u] == "dropout" && fld(u, "a") == P) { m.dropout = u; Pd = O(u).at("out").i32(); break; }
    for (int u : consumers_[Pd])
      if (kinds_[u] == "matmul_batched" && fld(u, "a") == Pd) { m.pv = u; break; }
    if (m.pv < 0) continue;
    const int q = fld((int)i, "a"), kt = fld((int)i, "b"), v = fld(m.pv, "b"), o = O(m.pv).at("out").i32();
    const View &vq = view_[q], &vk = view_[kt], &vv = view_[v], &vo = view_[o];
    if (vq.dims.size() != 4 || vk.dims.size() != 4 || vv.dims.size() != 4 || vo.dims.size() != 4) continue;
    const int64_t B = vq.dims[0], H = vq.dims[1], T = vq.dims[2], dh = vq.dims[3];
    if (!tgk::attention_supported(T, dh)) continue;
    if (vk.dims != Dims({B, H, dh, T}) || vv.dims != Dims({B, H, T, dh}) || vo.dims != Dims({B, H, T, dh})) continue;
    if (vq.strides[3] != 1 || vk.strides[2] != 1 || vv.strides[3] != 1 || vo.strides[3] != 1) continue;
    // 16-byte aligned rows (the stride of a size-1 dimension never moves the address)
    auto al4 = [](const View& w, int d) { return w.dims[d] == 1 || w.strides[d] % 4 == 0; };
    bool al = true;
    for (int d = 0; d < 3; ++d) al = al && al4(vq, d) && al4(vv, d);
    al = al && al4(vk, 0) && al4(vk, 1) && al4(vk, 3);
    if (!al) continue;
    if (view_[P].root != P || !view_[P].contiguous() || view_[Pd].root != Pd || !view_[Pd].contiguous()) continue;
    auto ready = [&](int t) {   // data of t exists before op i runs
      const int src = T_[view_[t].root].src;
      return src < 0 || src < (int)i || is_leaf(src);
    };
    if (!ready(v) || (m.dropout >= 0 && !ready(fld(m.dropout, "seed")))) continue;
    bool taken = false;
    for (int op : {m.qk, m.scale, m.softmax, m.dropout, m.pv}) if (op >= 0 && attn_of_[op] >= 0) taken = true;
    if (taken) continue;
    const int id = (int)attn_.size();
    attn_.push_back(m);
    for (int op : {m.qk, m.scale, m.softmax, m.dropout, m.pv}) if (op >= 0) attn_of_[op] = id;
  }
}

void Runtime::match_colsums() {
  colsum_.clear();
  colsum_done_.assign(ops_.size(), false);
  mul_absorbed_.assign(ops_.size(), false);
  auto pinned = [&](int t) {
    for (int o : outputs_) if (o == t) return true;
    for (auto& c : captures_) if (c.second == t) return true;
    for (auto& w : copy_writebacks_) if (w.first == t) return true;
    return false;
  };
  for (size_t i = 0; i < ops_.size(); ++i) {
    if (kinds_[i] != "sum_to_shape" || virtual_[i] || attn_of_[i] >= 0) continue;
    const int a = fld((int)i, "a"), out = O((int)i).at("out").i32();
    if (!view_[a].contiguous() || T_[a].dt != F32) continue;
    const Dims& as = T_[a].shape;
    const Dims& os = T_[out].shape;
    // target = [1.., kept suffix of as]: reduced dims form a leading block
    const int rdiff = (int)as.size() - (int)os.size();
    if (rdiff < 0) continue;
    size_t lead = 0;   // dims of `as` summed over
    bool ok = true, in_kept = false;
    for (size_t d = 0; d < as.size(); ++d) {
      const bool reduced = (int)d < rdiff || (os[d - rdiff] == 1 && as[d] != 1);
      if (reduced && in_kept) { ok = false; break; }
      if (!reduced && as[d] != 1) in_kept = true;
      if (reduced) lead = d + 1;
    }
    if (!ok) continue;
    int64_t R = 1, C = 1;
    for (size_t d = 0; d < as.size(); ++d) (d < lead ? R : C) *= as[d];
    if (R <= 1 || C <= 0 || C != T_[out].numel) continue;
    ColSumOp c{a, -1, R, C};
    const int m = T_[a].src;
    if (m >= 0 && kinds_[m] == "mul" && view_[a].root == a && consumers_[a].size() == 1 && !pinned(a) &&
        attn_of_[m] < 0) {
      const int x = fld(m, "a"), y = fld(m, "b");
      if (T_[x].dt == F32 && T_[y].dt == F32 && T_[x].shape == as && T_[y].shape == as && view_[x].contiguous() &&
          view_[y].contiguous()) {
        c.a = x;
        c.b = y;
        mul_absorbed_[m] = true;
      }
    }
    colsum_[(int)i] = c;
  }
}

// Op index at whose position op's node runs (its group's first op, its attention chain's
// first product, or itself).
int Runtime::emit_pos(int op) const {
  if (group_of_[op] >= 0) return groups_[group_of_[op]].first;
  if (attn_of_[op] >= 0)
    return attn_of_[op] < (int)attn_.size() ? attn_[attn_of_[op]].qk : attn_bwd_[attn_of_[op] - attn_.size()].first;
  return op;
}

void Runtime::lower_colsums(int s0) {
  std::vector<int> batch{s0};
  const ColSumOp& c0 = colsum_.at(s0);
  auto ready = [&](int t) {   // t's data exists before op s0's node runs
    const int p = T_[view_[t].root].src;
    if (p < 0 || is_leaf(p)) return true;
    if (colsum_.count(p)) return (bool)colsum_done_[p];
    if (mul_absorbed_[p]) return false;
    return emit_pos(p) < s0;
  };
  for (auto it = colsum_.upper_bound(s0); it != colsum_.end() && (int)batch.size() < tgk::kColSumMax; ++it) {
    const ColSumOp& c = it->second;
    if (colsum_done_[it->first] || defer_colsum_[it->first] || c.R != c0.R || c.C != c0.C) continue;
    if (!ready(c.a) || (c.b >= 0 && !ready(c.b))) continue;
    batch.push_back(it->first);
  }
  emit_colsums(batch);
}

bool Runtime::tail_rowsum(int gi, DeferredRowSum& d) const {
  const Group& G = groups_[gi];
  if (!G.row || !G.dups.empty() || G.ops.empty() || G.ops.size() > 2 || G.shape.empty()) return false;
  const int m0 = G.ops[0];
  const std::string& k0 = kinds_[m0];
  if (k0 != "sum_last" && k0 != "mean_last") return false;
  const int a = fld(m0, "a");
  const int s0 = O(m0).at("out").i32();
  const int64_t D = G.shape.back();
  if (D < 1 || T_[a].dt != F32 || T_[a].numel != D || !view_[a].contiguous()) return false;
  int out = s0;
  double scale = 1.0;
  std::string detail = k0;
  if (G.ops.size() == 2) {
    const int m1 = G.ops[1];
    if (kinds_[m1] != "mul_scalar" || fld(m1, "a") != s0 || consumers_[s0].size() != 1) return false;
    out = O(m1).at("out").i32();
    scale = O(m1).at("scalar").num();
    detail += ",mul_scalar";
  }
  if (!consumers_[out].empty() || T_[out].numel != 1 || T_[out].dt != F32 || !view_[out].contiguous()) return false;
  bool is_out = false;
  for (int o : outputs_) if (root(o) == root(out)) is_out = true;
  for (auto& c : captures_) if (root(c.second) == root(out)) is_out = true;
  for (auto& w : copy_writebacks_) if (root(w.first) == root(out)) return false;
  if (!is_out) return false;
  d = DeferredRowSum{gi, a, out, D, k0 == "mean_last" ? (double)D : 1.0, scale, detail};
  return true;
}

void Runtime::emit_scatter(const DeferredScatter& sc) {
  Node n;
  n.kind = "scatter";
  n.op = sc.op;
  n.shape = sc.shape;
  n.reads.push_back(root(sc.idx));
  n.reads.push_back(root(sc.b));
  n.writes.push_back(root(sc.out));
  n.flops = 0;
  n.bytes = 4.0 * (sc.rows + sc.rows * sc.N + sc.V * sc.N);
  const int64_t wsb = tgk::scatter_workspace_bytes(sc.rows, sc.V, sc.N);
  workspace_bytes_ = std::max(workspace_bytes_, (size_t)wsb);
  n.ws = wsb > 0;
  n.bind = [=]() -> std::function<void(hipStream_t)> {
    const int32_t* pi = (const int32_t*)dptr(sc.idx);
    const float* pd = (const float*)dptr(sc.b);
    float* po = (float*)dptr(sc.out);
    void* work = cur_ws_;
    const int64_t rows = sc.rows, V = sc.V, N = sc.N;
    return [=](hipStream_t st) { tgk::scatter_rows(pi, rows, pd, V, N, po, work, st); };
  };
  add_node(std::move(n));
}

void Runtime::emit_colsums(const std::vector<int>& batch, bool with_scatter, bool with_rowsums, bool with_mids) {
  const int s0 = batch.front();
  const ColSumOp& c0 = colsum_.at(s0);
  for (int sop : batch) colsum_done_[sop] = true;
  Node n;
  n.kind = "reduce";
  n.op = s0;
  n.shape = "[" + std::to_string(c0.R) + "," + std::to_string(c0.C) + "] x" + std::to_string(batch.size());
  for (int sop : batch)
    if (colsum_.at(sop).R != c0.R || colsum_.at(sop).C != c0.C) { n.shape = std::to_string(batch.size()) + " column sums"; break; }
  size_t ws = 0;
  std::vector<size_t> ws_off;
  std::vector<int64_t> cbase;
  int cscale = 1;
  {
    std::vector<int64_t> cs, rs;
    std::vector<int> ts;
    for (int sop : batch) {
      const ColSumOp& c = colsum_.at(sop);
      const auto pt = colsum_part_.find(sop);
      cs.push_back(c.C);
      rs.push_back(pt != colsum_part_.end() ? pt->second.rows : c.R);
      ts.push_back(c.b >= 0 ? 2 : 1);
    }
    cscale = tgk::colsum_batch_scale(cs.data(), rs.data(), ts.data(), (int)batch.size());
  }
  for (int sop : batch) {
    const ColSumOp& c = colsum_.at(sop);
    const auto pt = colsum_part_.find(sop);
    const bool from_part = pt != colsum_part_.end();   // a GEMM epilogue's f64 partials
    const int64_t R = from_part ? pt->second.rows : c.R;
    if (!from_part) n.reads.push_back(root(c.a));
    if (c.b >= 0) n.reads.push_back(root(c.b));
    const int out = O(sop).at("out").i32();
    n.writes.push_back(root(out));
    n.bytes += from_part ? 8.0 * R * c.C + 4.0 * c.C : 4.0 * (c.R * c.C * (c.b >= 0 ? 2 : 1) + c.C);
    n.detail += std::string(n.detail.empty() ? "" : ",") +
                (c.b >= 0 ? "mul,sum_to_shape" : from_part ? "sum_partials" : "sum_to_shape");
    ws_off.push_back(ws);
    const int terms = c.b >= 0 ? 2 : 1;
    ws += ((size_t)tgk::colsum_workspace_doubles(c.C, R, terms, cscale) * 8 + 255) & ~(size_t)255;
    cbase.push_back(take_counters(tgk::colsum_counters(c.C, R, terms, cscale)));
  }
  const std::vector<DeferredRowSum> rsums = with_rowsums ? deferred_rowsum_ : std::vector<DeferredRowSum>{};
  std::vector<size_t> rws_off;
  std::vector<int64_t> rcbase;
  for (const DeferredRowSum& d : rsums) {
    n.reads.push_back(root(d.a));
    n.writes.push_back(root(d.out));
    n.bytes += 4.0 * (d.R + 1);
    n.detail += "," + d.detail;
    n.shape += " + loss [" + std::to_string(d.R) + "]";
    rws_off.push_back(ws);
    ws += ((size_t)tgk::colsum_workspace_doubles(1, d.R, 1) * 8 + 255) & ~(size_t)255;
    rcbase.push_back(take_counters(tgk::colsum_counters(1, d.R, 1)));
  }
  const std::vector<DeferredMidSum> mids = with_mids ? deferred_midsum_ : std::vector<DeferredMidSum>{};
  std::vector<size_t> mws_off;
  std::vector<int64_t> mcbase;
  for (const DeferredMidSum& d : mids) {
    n.reads.push_back(root(d.a));
    n.writes.push_back(root(d.out));
    n.bytes += 4.0 * (d.B * d.C * d.L + d.C);
    n.detail += ",sum_to_shape";
    n.shape += " + [" + std::to_string(d.B) + "," + std::to_string(d.C) + "," + std::to_string(d.L) + "] sum";
    mws_off.push_back(ws);
    ws += ((size_t)tgk::midsum_workspace_doubles(d.B, d.C, d.L) * 8 + 255) & ~(size_t)255;
    mcbase.push_back(take_counters(tgk::midsum_counters(d.B, d.C, d.L)));
  }
  workspace_bytes_ = std::max(workspace_bytes_, ws);
  n.ws = true;
  const bool sct = with_scatter && !deferred_scatter_.empty();
  const DeferredScatter sc = sct ? deferred_scatter_.front() : DeferredScatter{};
  size_t sws_off = 0;
  int64_t scbase = 0;
  if (sct) {
    n.reads.push_back(root(sc.idx));
    n.reads.push_back(root(sc.b));
    n.writes.push_back(root(sc.out));
    n.bytes += 4.0 * (sc.rows + sc.rows * sc.N + sc.V * sc.N);
    n.detail += ",scatter";
    n.shape += " + scatter " + sc.shape;
    sws_off = ws;
    ws += ((size_t)tgk::scatter_workspace_doubles(sc.rows, sc.V, sc.N) * 8 + 255) & ~(size_t)255;
    scbase = take_counters(tgk::scatter_counters(sc.rows, sc.V, sc.N));
    workspace_bytes_ = std::max(workspace_bytes_, ws);
  }
  n.bind = [=]() -> std::function<void(hipStream_t)> {
    tgk::ColSumBatch bt{};
    bt.n = (int)batch.size();
    if (sct) {
      if (T_[root(sc.b)].numel < sc.rows * sc.N || T_[root(sc.out)].numel < sc.V * sc.N ||
          T_[root(sc.idx)].numel < sc.rows)
        throw Error(TG_INTERNAL, "embedding gradient: operand smaller than its shape");
      bt.sc.idx = (const int32_t*)dptr(sc.idx);
      bt.sc.dy = (const float*)dptr(sc.b);
      bt.sc.out = (float*)dptr(sc.out);
      bt.sc.rows = sc.rows;
      bt.sc.N = sc.N;
      bt.sc.V = (int)sc.V;
      bt.sc.part = reinterpret_cast<double*>(reinterpret_cast<char*>(cur_ws_) + sws_off);
      bt.sc.counters = cur_counters_ + scbase;
    }
    for (size_t q = 0; q < batch.size(); ++q) {
      const ColSumOp& c = colsum_.at(batch[q]);
      const int out = O(batch[q]).at("out").i32();
      double* part = reinterpret_cast<double*>(reinterpret_cast<char*>(cur_ws_) + ws_off[q]);
      const auto pt = colsum_part_.find(batch[q]);
      if (pt != colsum_part_.end()) {
        if (T_[root(out)].numel < c.C || pt->second.off + (size_t)pt->second.rows * c.C * 8 > partial_bytes_)
          throw Error(TG_INTERNAL, "column sum: partials outside their region");
        bt.s[q] = tgk::colsum_desc_f64(reinterpret_cast<const double*>(partials_ + pt->second.off),
                                       (float*)dptr(out), c.C, pt->second.rows, part, cur_counters_ + cbase[q],
                                       cscale);
        continue;
      }
      if (T_[root(c.a)].numel < c.R * c.C || (c.b >= 0 && T_[root(c.b)].numel < c.R * c.C) ||
          T_[root(out)].numel < c.C)
        throw Error(TG_INTERNAL, "column sum: operand smaller than its shape");
      bt.s[q] = tgk::colsum_desc((const float*)dptr(c.a), c.b >= 0 ? (const float*)dptr(c.b) : nullptr,
                                 (float*)dptr(out), c.C, c.R, c.C, 1.0, part, cur_counters_ + cbase[q], cscale);
    }
    for (size_t q = 0; q < mids.size(); ++q) {
      const DeferredMidSum& d = mids[q];
      if (T_[root(d.a)].numel < d.B * d.C * d.L || T_[root(d.out)].numel < d.C)
        throw Error(TG_INTERNAL, "[B, C, L] sum: operand smaller than its shape");
      double* part = reinterpret_cast<double*>(reinterpret_cast<char*>(cur_ws_) + mws_off[q]);
      bt.m[bt.nmid++] = tgk::midsum_desc((const float*)dptr(d.a), (float*)dptr(d.out), d.B, d.C, d.L, part,
                                         cur_counters_ + mcbase[q]);
    }
    for (size_t q = 0; q < rsums.size(); ++q) {
      const DeferredRowSum& d = rsums[q];
      if (T_[root(d.a)].numel < d.R || T_[root(d.out)].numel < 1)
        throw Error(TG_INTERNAL, "loss sum: operand smaller than its shape");
      double* part = reinterpret_cast<double*>(reinterpret_cast<char*>(cur_ws_) + rws_off[q]);
      tgk::ColSum c = tgk::colsum_desc((const float*)dptr(d.a), nullptr, (float*)dptr(d.out), 1, d.R, 1, d.div, part,
                                       cur_counters_ + rcbase[q], 1);
      c.scale = d.scale;
      bt.s[bt.n++] = c;
    }
    return [bt](hipStream_t st) { tgk::colsum_batch(bt, st); };
  };
  add_node(std::move(n));
}

void Runtime::match_attention_bwd() {
  attn_bwd_.clear();
  if (attn_.empty()) return;
  auto pinned = [&](int t) {
    for (int o : outputs_) if (o == t) return true;
    for (auto& c : captures_) if (c.second == t) return true;
    for (auto& w : copy_writebacks_) if (w.first == t) return true;
    return false;
  };
  auto out_of = [&](int op) { return O(op).at("out").i32(); };
  auto only = [&](int t) { return consumers_[t].size() == 1 ? consumers_[t][0] : -1; };
  // v is a transpose (last two dims) of u, over the same storage (strides of size-1
  // dimensions do not matter)
  auto transposed = [&](int v, int u) {
    const View &a = view_[v], &b = view_[u];
    if (a.root != b.root || a.dims.size() != 4 || b.dims.size() != 4) return false;
    static const int perm[4] = {0, 1, 3, 2};
    for (int d = 0; d < 4; ++d)
      if (a.dims[d] != b.dims[perm[d]] || (a.dims[d] != 1 && a.strides[d] != b.strides[perm[d]])) return false;
    return true;
  };
  auto is_mul_of = [&](int op, int x, int y) {   // op = x * y (either order), f32
    if (op < 0 || kinds_[op] != "mul") return false;
    const int a = fld(op, "a"), b = fld(op, "b");
    return (a == x && b == y) || (a == y && b == x);
  };
  for (size_t f = 0; f < attn_.size(); ++f) {
    const AttnMatch& m = attn_[f];
    const int q = fld(m.qk, "a"), kt = fld(m.qk, "b"), v = fld(m.pv, "b");
    const int P = out_of(m.softmax);
    const int Pd = m.dropout >= 0 ? out_of(m.dropout) : P;
    AttnBwd bw{(int)f, -1, -1, -1, -1, -1, -1, {}};
    // dPd = dO @ V^T
    int dO = -1;
    for (size_t i = 0; i < ops_.size() && bw.dpd < 0; ++i) {
      if (kinds_[i] != "matmul_batched" || attn_of_[i] >= 0 || virtual_[i]) continue;
      if (transposed(fld((int)i, "b"), v)) { bw.dpd = (int)i; dO = fld((int)i, "a"); }
    }
    if (bw.dpd < 0) continue;
    const View& vo = view_[dO];
    auto al4 = [](const View& w, int d) { return w.dims[d] == 1 || w.strides[d] % 4 == 0; };
    if (vo.dims != view_[v].dims || vo.strides[3] != 1 || !al4(vo, 0) || !al4(vo, 1) || !al4(vo, 2)) continue;
    std::vector<int> chain{bw.dpd};
    int dP = out_of(bw.dpd);
    if (pinned(dP)) continue;
    if (m.dropout >= 0) {
      const int d = only(dP);
      if (d < 0 || kinds_[d] != "dropout" || fld(d, "seed") != fld(m.dropout, "seed") ||
          O(d).at("salt").i64() != O(m.dropout).at("salt").i64() || O(d).at("p").num() != O(m.dropout).at("p").num())
        continue;
      chain.push_back(d);
      dP = out_of(d);
      if (pinned(dP)) continue;
    }
    // softmax backward: s1 = dP - broadcast(reshape(sum_last(dP * P))), dS = s1 * P [* scale]
    if (consumers_[dP].size() != 2) continue;
    int m1 = -1, s1 = -1;
    for (int c : consumers_[dP]) {
      if (is_mul_of(c, dP, P)) m1 = c;
      else if (kinds_[c] == "sub" && fld(c, "a") == dP) s1 = c;
    }
    if (m1 < 0 || s1 < 0 || pinned(out_of(m1))) continue;
    const int r1 = only(out_of(m1));
    if (r1 < 0 || kinds_[r1] != "sum_last" || pinned(out_of(r1))) continue;
    const int rs = only(out_of(r1));
    if (rs < 0 || kinds_[rs] != "reshape" || pinned(out_of(rs))) continue;
    const int bc = only(out_of(rs));
    if (bc < 0 || kinds_[bc] != "broadcast_to" || pinned(out_of(bc)) || only(out_of(bc)) != s1 ||
        fld(s1, "b") != out_of(bc))
      continue;
    const int m2 = only(out_of(s1));
    if (!is_mul_of(m2, out_of(s1), P) || pinned(out_of(s1))) continue;
    chain.insert(chain.end(), {m1, r1, rs, bc, s1, m2});
    int dS = out_of(m2);
    if (m.scale >= 0) {
      const int ms = only(dS);
      if (ms < 0 || kinds_[ms] != "mul_scalar" || O(ms).at("scalar").num() != O(m.scale).at("scalar").num() ||
          pinned(dS))
        continue;
      chain.push_back(ms);
      dS = out_of(ms);
      bw.ds_op = ms;
    } else {
      bw.ds_op = m2;
    }
    if (pinned(dS) || consumers_[dS].size() != 2) continue;
    for (int c : consumers_[dS]) {
      if (kinds_[c] != "matmul_batched" || attn_of_[c] >= 0) continue;
      if (fld(c, "a") == dS && transposed(fld(c, "b"), kt)) bw.dq = c;
      else if (fld(c, "b") == dS && transposed(fld(c, "a"), q)) bw.dkt = c;
    }
    if (bw.dq < 0 || bw.dkt < 0) continue;
    // dV = Pd^T dO
    for (int c : consumers_[dO])
      if (kinds_[c] == "matmul_batched" && attn_of_[c] < 0 && fld(c, "b") == dO && transposed(fld(c, "a"), Pd))
        bw.dv = c;
    if (bw.dv < 0) continue;
    const View &vq = view_[out_of(bw.dq)], &vk = view_[out_of(bw.dkt)], &vv = view_[out_of(bw.dv)];
    if (vq.strides[3] != 1 || vv.strides[3] != 1 || vq.dims != vo.dims || vv.dims != vo.dims ||
        vk.dims != view_[kt].dims)
      continue;
    chain.insert(chain.end(), {bw.dq, bw.dkt, bw.dv});
    bool free_ops = true;
    for (int op : chain) if (attn_of_[op] >= 0) free_ops = false;
    if (!free_ops) continue;
    bw.first = *std::min_element(chain.begin(), chain.end());
    // everything the node reads exists at its position
    auto ready = [&](int t) {
      const int src = T_[view_[t].root].src;
      return src < 0 || is_leaf(src) || src < bw.first;
    };
    if (!ready(dO)) continue;
    bw.ops = chain;
    const int id = (int)(attn_.size() + attn_bwd_.size());
    attn_bwd_.push_back(bw);
    for (int op : chain) attn_of_[op] = id;
  }
}

void Runtime::lower_attention_bwd(int bi) {
  const AttnBwd bw = attn_bwd_[bi];
  const AttnMatch m = attn_[bw.fwd];
  auto out_of = [&](int op) { return O(op).at("out").i32(); };
  const int q = fld(m.qk, "a"), kt = fld(m.qk, "b"), v = fld(m.pv, "b");
  const int P = out_of(m.softmax);
  const int Pd = m.dropout >= 0 ? out_of(m.dropout) : P;
  const int dO = fld(bw.dpd, "a");
  const int dS = out_of(bw.ds_op), dQ = out_of(bw.dq), dKt = out_of(bw.dkt), dV = out_of(bw.dv);
  const int seed = m.dropout >= 0 ? fld(m.dropout, "seed") : -1;
  const View vq = view_[q], vk = view_[kt], vv = view_[v], vo = view_[dO];
  const View wq = view_[dQ], wk = view_[dKt], wv = view_[dV];
  const int64_t B = vq.dims[0], H = vq.dims[1], T = vq.dims[2], dh = vq.dims[3];
  Node n;
  n.kind = "attention";
  n.op = bw.first;
  n.shape = shape_str(vq.dims) + " T=" + std::to_string(T) + " backward";
  n.detail = "attention_backward";
  for (int t : {q, kt, v, P, Pd, dO}) n.reads.push_back(root(t));
  if (seed >= 0) n.reads.push_back(root(seed));
  for (int t : {dS, dQ, dKt, dV}) n.writes.push_back(root(t));
  n.flops = 8.0 * (double)B * H * T * T * dh;
  n.bytes = 4.0 * (double)B * H * T * (8 * dh + 4 * T);
  const double scale = m.scale >= 0 ? O(m.scale).at("scalar").num() : 1.0;
  double dp = 0, dsc = 1;
  uint32_t salt = 0;
  if (m.dropout >= 0) {
    dp = O(m.dropout).at("p").num();
    dsc = 1.0 / (1.0 - dp);
    salt = (uint32_t)(uint64_t)std::fmod((double)O(m.dropout).at("salt").i64() * 2654435761.0, 4294967296.0);
  }
  n.bind = [=]() -> std::function<void(hipStream_t)> {
    {
      int64_t d4[4] = {B, H, T, dh}, dt[4] = {B, H, dh, T};
      check_span("attention bwd dO", T_[root(dO)].numel, 0, d4, vo.strides.data(), 4);
      check_span("attention bwd dQ", T_[root(dQ)].numel, 0, d4, wq.strides.data(), 4);
      check_span("attention bwd dK", T_[root(dKt)].numel, 0, dt, wk.strides.data(), 4);
      check_span("attention bwd dV", T_[root(dV)].numel, 0, d4, wv.strides.data(), 4);
      if (T_[root(dS)].numel < B * H * T * T || !view_[dS].contiguous() || view_[dS].root != dS)
        throw Error(TG_INTERNAL, "attention backward: dS must be a contiguous [B, H, T, T] tensor");
    }
    tgk::AttnBwdDesc a{};
    a.B = (int)B; a.H = (int)H; a.T = (int)T; a.dh = (int)dh;
    a.dout = (const float*)dptr(dO); a.sob = vo.strides[0]; a.soh = vo.strides[1]; a.soi = vo.strides[2];
    a.q = (const float*)dptr(q); a.sqb = vq.strides[0]; a.sqh = vq.strides[1]; a.sqi = vq.strides[2];
    a.k = (const float*)dptr(kt); a.skb = vk.strides[0]; a.skh = vk.strides[1]; a.skj = vk.strides[3];
    a.v = (const float*)dptr(v); a.svb = vv.strides[0]; a.svh = vv.strides[1]; a.svj = vv.strides[2];
    a.p = (const float*)dptr(P);
    a.pd = (const float*)dptr(Pd);
    a.ds = (float*)dptr(dS);
    a.dq = (float*)dptr(dQ); a.sdqb = wq.strides[0]; a.sdqh = wq.strides[1]; a.sdqi = wq.strides[2];
    a.dk = (float*)dptr(dKt); a.sdkb = wk.strides[0]; a.sdkh = wk.strides[1]; a.sdkj = wk.strides[3];
    a.sdkd = wk.strides[2];
    a.dv = (float*)dptr(dV); a.sdvb = wv.strides[0]; a.sdvh = wv.strides[1]; a.sdvj = wv.strides[2];
    a.has_scale = m.scale >= 0;
    a.scale = scale;
    a.has_dropout = m.dropout >= 0;
    a.drop_p = dp;
    a.drop_scale = dsc;
    a.salt = salt;
    a.seed = seed >= 0 ? (const int32_t*)dptr(seed) : nullptr;
    return [a](hipStream_t st) { tgk::attention_bwd(a, st); };
  };
  add_node(std::move(n));
}

void Runtime::lower_attention(int mi) {
  const AttnMatch m = attn_[mi];
  const int q = fld(m.qk, "a"), kt = fld(m.qk, "b"), v = fld(m.pv, "b"), o = O(m.pv).at("out").i32();
  const int P = O(m.softmax).at("out").i32();
  const int Pd = m.dropout >= 0 ? O(m.dropout).at("out").i32() : -1;
  const int seed = m.dropout >= 0 ? fld(m.dropout, "seed") : -1;
  const View vq = view_[q], vk = view_[kt], vv = view_[v], vo = view_[o];
  const int64_t B = vq.dims[0], H = vq.dims[1], T = vq.dims[2], dh = vq.dims[3];
  Node n;
  n.kind = "attention";
  n.op = m.qk;
  n.shape = shape_str(vq.dims) + " T=" + std::to_string(T);
  n.detail = std::string("matmul_batched") + (m.scale >= 0 ? ",mul_scalar" : "") + ",softmax_causal_last" +
             (m.dropout >= 0 ? ",dropout" : "") + ",matmul_batched";
  for (int t : {q, kt, v}) n.reads.push_back(root(t));
  if (seed >= 0) n.reads.push_back(root(seed));
  n.writes.push_back(root(P));
  if (Pd >= 0) n.writes.push_back(root(Pd));
  n.writes.push_back(root(o));
  n.flops = 4.0 * (double)B * H * T * T * dh;
  n.bytes = 4.0 * (double)B * H * T * (4 * dh + (Pd >= 0 ? 2 : 1) * T);
  const double scale = m.scale >= 0 ? O(m.scale).at("scalar").num() : 1.0;
  double dp = 0, dsc = 1;
  uint32_t salt = 0;
  if (m.dropout >= 0) {
    dp = O(m.dropout).at("p").num();
    dsc = 1.0 / (1.0 - dp);
    salt = (uint32_t)(uint64_t)std::fmod((double)O(m.dropout).at("salt").i64() * 2654435761.0, 4294967296.0);
  }
  n.bind = [=]() -> std::function<void(hipStream_t)> {
    {
      int64_t dq[4] = {B, H, T, dh}, dk[4] = {B, H, dh, T}, dd[4] = {B, H, T, dh};
      check_span("attention q", T_[root(q)].numel, 0, dq, vq.strides.data(), 4);
      check_span("attention k", T_[root(kt)].numel, 0, dk, vk.strides.data(), 4);
      check_span("attention v", T_[root(v)].numel, 0, dd, vv.strides.data(), 4);
      check_span("attention o", T_[root(o)].numel, 0, dd, vo.strides.data(), 4);
      if (T_[root(P)].numel < B * H * T * T || (Pd >= 0 && T_[root(Pd)].numel < B * H * T * T))
        throw Error(TG_INTERNAL, "attention: probability tensor too small");
    }
    tgk::AttnDesc a{};
    a.B = (int)B; a.H = (int)H; a.T = (int)T; a.dh = (int)dh;
    a.q = (const float*)dptr(q); a.sqb = vq.strides[0]; a.sqh = vq.strides[1]; a.sqi = vq.strides[2];
    a.k = (const float*)dptr(kt); a.skb = vk.strides[0]; a.skh = vk.strides[1]; a.skj = vk.strides[3];
    a.v = (const float*)dptr(v); a.svb = vv.strides[0]; a.svh = vv.strides[1]; a.svj = vv.strides[2];
    a.o = (float*)dptr(o); a.sob = vo.strides[0]; a.soh = vo.strides[1]; a.soi = vo.strides[2];
    a.p = (float*)dptr(P);
    a.pd = Pd >= 0 ? (float*)dptr(Pd) : nullptr;
    a.has_scale = m.scale >= 0;
    a.scale = scale;
    a.has_dropout = m.dropout >= 0;
    a.drop_p = dp;
    a.drop_scale = dsc;
    a.salt = salt;
    a.seed = seed >= 0 ? (const int32_t*)dptr(seed) : nullptr;
    return [a](hipStream_t st) { tgk::attention_fwd(a, st); };
  };
  add_node(std::move(n));
}

void Runtime::check_gemm_spans(const tgk::GemmDesc& d, int a, int b, int out) const {
  int64_t nb0 = d.batch / d.bdiv;
  int64_t da[4] = {nb0, d.bdiv, d.M, d.K}, sa[4] = {d.sAz0, d.sAz1, d.sAm, d.sAk};
  int64_t db[4] = {nb0, d.bdiv, d.K, d.N}, sb[4] = {d.sBz0, d.sBz1, d.sBk, d.sBn};
  int64_t dc[4] = {nb0, d.bdiv, d.M, d.N}, sc[4] = {d.sCz0, d.sCz1, d.sCm, d.sCn};
  if (d.batch % d.bdiv != 0) throw Error(TG_INTERNAL, "gemm: batch not divisible by bdiv");
  check_span("gemm A", T_[root(a)].numel, 0, da, sa, 4);
  check_span("gemm B", T_[root(b)].numel, 0, db, sb, 4);
  check_span("gemm C", T_[root(out)].numel, 0, dc, sc, 4);
  if (d.batch * d.M * d.N != T_[out].numel) throw Error(TG_INTERNAL, "gemm: output size mismatch");
}

// True when every reader of tensor t (through views) is an op of the fused optimizer and t
// is no output, capture or writeback source.
bool Runtime::only_optimizer_reads(int t) const {
  for (int o : outputs_) if (root(o) == root(t)) return false;
  for (auto& c : captures_) if (root(c.second) == root(t)) return false;
  for (auto& w : copy_writebacks_) if (root(w.first) == root(t)) return false;
  if (consumers_[t].empty()) return false;
  for (int c : consumers_[t]) {
    if (adam_ops_.count(c)) continue;
    // views of t (a product with an identity one-hot is one; products lowered by other
    // patterns are not)
    const bool view = (kinds_[c] != "matmul" && kinds_[c] != "matmul_batched") || root(O(c).at("out").i32()) == root(t);
    if (virtual_[c] && !is_leaf(c) && view) {
      if (!only_optimizer_reads(O(c).at("out").i32())) return false;
      continue;
    }
    return false;
  }
  return true;
}

// Candidates: split-K GEMMs read only by the fused optimizer. A kind's candidates are
// grouped when their whole-K 64 x 64 tiles fill the chip at least once (256 CUs);
// fewer, longer tiles would leave CUs idle, so such GEMMs keep their split-K launches.
void Runtime::plan_gemm_groups() {
  defer_gemm_.assign(ops_.size(), 0);
  if (!use_gemm_group_) return;
  std::vector<int> cand[4];
  int64_t tiles[4] = {0, 0, 0, 0};
  for (size_t i = 0; i < ops_.size(); ++i) {
    if ((kinds_[i] != "matmul" && kinds_[i] != "matmul_batched") || virtual_[i]) continue;
    const int a = fld((int)i, "a"), b = fld((int)i, "b");
    if (kinds_[T_[view_[a].root].src] == "one_hot" || kinds_[T_[view_[b].root].src] == "one_hot") continue;
    tgk::GemmDesc d{};
    if (!gemm_desc((int)i, d) || tgk::gemm_workspace_floats(d) <= 0) continue;
    if (!only_optimizer_reads(O((int)i).at("out").i32())) continue;
    const int kind = tgk::gemm_group_kind(d);
    if (kind < 0) continue;
    cand[kind].push_back((int)i);
    tiles[kind] += ((d.M + 63) / 64) * ((d.N + 63) / 64) * d.batch;
  }
  for (int k = 0; k < 4; ++k)
    if (tiles[k] >= 256)
      for (int i : cand[k]) defer_gemm_[i] = 1;
}

int Runtime::epi_group(int op, int out, const tgk::GemmDesc& d, bool& store_c, const CatFwd* cat) const {
  store_c = false;
  if (view_[out].root != out || !view_[out].contiguous() || d.batch != 1 || d.sCn != 1 || d.sCm != d.N) return -1;
  for (int o : outputs_) if (root(o) == out) store_c = true;
  for (auto& c : captures_) if (root(c.second) == out) store_c = true;
  for (auto& w : copy_writebacks_) if (root(w.first) == out) store_c = true;
  // The element group that reads the product first (through views). Any other reader
  // (another group, one that recomputes a member, a GEMM) reads the product from memory,
  // which the epilogue then stores too.
  int gi = -1;
  std::vector<int> stack{out};
  while (!stack.empty()) {
    const int t = stack.back();
    stack.pop_back();
    for (int c : consumers_[t]) {
      if (virtual_[c] && (kinds_[c] == "reshape" || kinds_[c] == "stop_gradient" || kinds_[c] == "slice_range")) {
        stack.push_back(O(c).at("out").i32());
        continue;
      }
      const int g = group_of_[c];
      for (size_t q = 0; q < groups_.size(); ++q)
        if ((int)q != g && dup_in((int)q, c)) store_c = true;   // q evaluates c again
      if (g < 0 || dropped_[c]) { store_c = true; continue; }
      if (gi < 0 || g == gi) { gi = g; continue; }
      store_c = true;
      if (groups_[g].first < groups_[gi].first) gi = g;
    }
  }
  if (gi < 0 || group_done_[gi] || groups_[gi].row || groups_[gi].first <= op || !groups_[gi].dups.empty()) return -1;
  const Group& G = groups_[gi];
  if (prod(G.shape) != d.M * d.N) return -1;
  tgk::GemmEpiCfg c{};
  tgk::gd::GemmArgs ga{};
  int64_t blocks = 0;
  if (cat) {
    const tgk::GemmCat gc{nullptr, cat->k0, cat->k1};
    if (!tgk::gemm_cat_epi_cfg(d, gc, c, ga, blocks)) return -1;
  } else if (tgk::gemm_workspace_floats(d) != 0 || !tgk::gemm_epi_cfg(d, c, ga, blocks)) {
    return -1;
  }
  const GroupPlan gp = plan_group(G.ops, false, G.shape);
  int hits = 0;
  for (auto& e : gp.ext) {
    if (root(e.first) == out) {
      // read whole and in order: a view of the full product with the group's shape
      if (T_[e.first].numel != T_[out].numel || !view_[e.first].contiguous() || T_[e.first].shape != G.shape) return -1;
      ++hits;
    } else if (!ready_now(e.first) && !const_early_ok(e.first)) {
      return -1;
    }
  }
  if (hits != 1 || (gp.seed >= 0 && !ready_now(gp.seed))) return -1;
  return gi;
}

bool Runtime::epi_cheap(int gi) const {
  static const std::set<std::string> costly = {"erf", "tanh", "sigmoid", "sin", "cos", "exp", "log", "rsqrt", "dropout"};
  for (int m : groups_[gi].ops)
    if (costly.count(kinds_[m])) return false;
  for (int m : groups_[gi].dups)
    if (costly.count(kinds_[m])) return false;
  return true;
}

void Runtime::lower_gemm_epi(int op, const tgk::GemmDesc& d, int a, int b, int out, int gi, bool store_c,
                             const CatFwd* cat) {
  const bool is_cat = cat != nullptr;
  const CatFwd cf = is_cat ? *cat : CatFwd{-1, -1, 0, 0};
  group_done_[gi] = 1;
  const Group G = groups_[gi];
  const GroupPlan gp = plan_group(G.ops, false, G.shape);
  // constants the group reads that are not lowered yet: lowered now, ahead of their position
  for (auto& e : gp.ext)
    if (root(e.first) != out && !ready_now(e.first)) lower_const_early(e.first);
  Node n;
  n.kind = "gemm";
  n.op = op;
  n.detail = "gemm+";
  for (size_t q = 0; q < G.ops.size(); ++q) n.detail += (q ? "," : "") + kinds_[G.ops[q]];
  n.shape = shape_str(T_[out].shape) + " x" + std::to_string(G.ops.size());
  if (is_cat) {
    n.detail = "gemm_cat+" + n.detail.substr(5);
    n.reads.push_back(root(cf.src0));
    n.reads.push_back(root(cf.src1));
  } else {
    n.reads.push_back(root(a));
  }
  n.reads.push_back(root(b));
  for (auto& e : gp.ext) if (root(e.first) != out) n.reads.push_back(root(e.first));
  if (gp.seed >= 0) n.reads.push_back(root(gp.seed));
  for (int t : gp.outs) n.writes.push_back(root(t));
  if (store_c) n.writes.push_back(root(out));
  n.flops = 2.0 * (double)d.M * d.N * d.K * d.batch;
  n.bytes = 4.0 * ((double)T_[a].numel + T_[b].numel) + (store_c ? 4.0 * T_[out].numel : 0.0);
  for (auto& e : gp.ext) if (root(e.first) != out) n.bytes += 4.0 * T_[e.first].numel;
  for (int t : gp.outs) n.bytes += 4.0 * T_[t].numel;
  // A deferred column sum of one of the group's outputs over all of the product's rows:
  // the epilogue also writes that output's column partials (one f64 row per tile row slot
  // of wavefronts), which the column-sum launch adds instead of reading the output back.
  int cs_out = -1, cs_op = -1;
  size_t cs_off = 0;
  if (use_colsum_epi_ && any_deferred_colsum_ && d.batch == 1) {
    for (size_t q = 0; q < gp.outs.size() && cs_op < 0; ++q) {
      const int t = gp.outs[q];
      if (T_[t].dt != F32 || T_[t].numel != d.M * d.N || !view_[t].contiguous()) continue;
      for (const auto& kv : colsum_) {
        const ColSumOp& so = kv.second;
        if (root(so.a) != root(t) || T_[so.a].numel != T_[t].numel || !view_[so.a].contiguous() || so.b >= 0 ||
            so.C != d.N || so.R != d.M || !defer_colsum_[kv.first] || colsum_done_[kv.first] ||
            colsum_part_.count(kv.first))
          continue;
        cs_op = kv.first;
        cs_out = (int)q;
        break;
      }
    }
    if (cs_op >= 0) {
      tgk::GemmEpiCfg c{};
      tgk::gd::GemmArgs ga{};
      int64_t blocks = 0;
      const bool ok = is_cat ? tgk::gemm_cat_epi_cfg(d, tgk::GemmCat{nullptr, cf.k0, cf.k1}, c, ga, blocks)
                             : tgk::gemm_epi_cfg(d, c, ga, blocks);
      if (!ok) throw Error(TG_INTERNAL, "GEMM epilogue: no direct-to-LDS launch");
      if (c.tiny || c.skinny) {   // these kernels write no column partials
        cs_op = cs_out = -1;
      } else {
        const int64_t rows = tgk::gemm_epi_colsum_rows(c, ga);
        cs_off = take_partials((size_t)rows * (size_t)d.N * 8);
        colsum_part_[cs_op] = ColPart{cs_off, rows};
        n.bytes += 8.0 * (double)rows * (double)d.N;
        n.detail += ",colsum";
      }
    }
  }
  const size_t code_off = fused_code_.size();
  fused_code_.insert(fused_code_.end(), gp.code.begin(), gp.code.end());
  n.bind = [=]() -> std::function<void(hipStream_t)> {
    if (is_cat) check_cat_spans(d, cf, b, out, store_c);
    else check_gemm_spans(d, a, b, out);
    const Dims F = G.shape;
    const int64_t cnt = prod(F);
    if (cnt >= (int64_t(1) << 31)) throw Error(TG_INVALID_ARGUMENT, "GEMM epilogue: 2^31 or more elements");
    // The group's element program, one element per call: operands by their broadcast
    // strides over F (merged dims), the product as input h_in.
    tgk::FusedProgram p;
    memset(&p, 0, sizeof(p));
    const size_t nx = gp.ext.size();
    std::vector<Dims> bs(nx, Dims(F.size(), 0));
    for (size_t q = 0; q < nx; ++q) {
      const View& v = view_[gp.ext[q].first];
      const int off = (int)F.size() - (int)v.dims.size();
      if (off < 0 || gp.ext[q].second != 0) throw Error(TG_INTERNAL, "GEMM epilogue: operand class");
      for (size_t dd = 0; dd < v.dims.size(); ++dd) bs[q][off + dd] = v.dims[dd] == 1 ? 0 : v.strides[dd];
      check_span("epilogue operand", T_[v.root].numel, 0, F.data(), bs[q].data(), (int)F.size());
    }
    Dims md;
    std::vector<Dims> ms(nx);
    for (size_t dd = 0; dd < F.size(); ++dd) {
      if (F[dd] == 1) continue;
      bool merge = !md.empty();
      for (size_t q = 0; q < nx && merge; ++q) merge = ms[q].back() == bs[q][dd] * F[dd];
      if (merge) {
        md.back() *= F[dd];
        for (size_t q = 0; q < nx; ++q) ms[q].back() = bs[q][dd];
      } else {
        md.push_back(F[dd]);
        for (size_t q = 0; q < nx; ++q) ms[q].push_back(bs[q][dd]);
      }
    }
    if (md.empty()) { md.push_back(1); for (auto& m : ms) m.push_back(0); }
    if (md.size() > (size_t)tgk::kMaxRank) throw Error(TG_INTERNAL, "GEMM epilogue: rank too large");
    const int R = (int)md.size();
    const Dims cs = contiguous_strides(md);
    p.n_in = (int)nx;
    p.nregs = gp.nregs;
    p.vec = 1;
    p.rank = R;
    for (int dd = 0; dd < R; ++dd) p.div[dd] = tgk::make_fastdiv((uint32_t)md[dd]);
    int h_in = -1;
    for (size_t q = 0; q < nx; ++q) {
      const View& v = view_[gp.ext[q].first];
      bool contig = true, scalar = true;
      for (int dd = 0; dd < R; ++dd) {
        if (ms[q][dd] != cs[dd]) contig = false;
        if (ms[q][dd] != 0) scalar = false;
      }
      const int m = contig ? tgk::FM_CONTIG : (scalar ? tgk::FM_SCALAR : tgk::FM_STRIDED);
      if (v.root == out) {
        // (a one-element product merges to no dimension and reads as a scalar: the same element)
        if (m != tgk::FM_CONTIG && cnt != 1) throw Error(TG_INTERNAL, "GEMM epilogue: the product is not read in order");
        h_in = (int)q;
      }
      p.in[q] = ptr_[v.root];
      p.in_dt[q] = kdt(T_[gp.ext[q].first].dt);
      p.in_mode[q] = m;
      p.in_inner[q] = (int32_t)ms[q][R - 1];
      if (m == tgk::FM_STRIDED) p.any_strided = 1;
      for (int dd = 0; dd < R; ++dd) p.in_strides[q][dd] = (int32_t)ms[q][dd];
    }
    p.n_out = (int)gp.outs.size();
    for (size_t q = 0; q < gp.outs.size(); ++q) {
      const int t = gp.outs[q];
      p.out[q] = dptr(t);
      p.out_dt[q] = kdt(T_[t].dt);
      p.out_reg[q] = gp.out_reg[q];
      if (T_[root(t)].numel < cnt || T_[t].numel != cnt || !view_[t].contiguous())
        throw Error(TG_INTERNAL, "GEMM epilogue: output size mismatch");
    }
    p.seed = gp.seed >= 0 ? (const int32_t*)dptr(gp.seed) : nullptr;
    p.n_instr = (int)gp.code.size();
    tgk::GemmDesc e = d;
    e.A = (const float*)dptr(is_cat ? cf.src0 : a);
    e.B = (const float*)dptr(b);
    e.C = store_c ? (float*)dptr(out) : nullptr;   // stored only when something else reads it
    tgk::GemmEpiCfg c{};
    tgk::gd::GemmArgs ga{};
    int64_t blocks = 0;
    if (is_cat) {
      const tgk::GemmCat gc{(const float*)dptr(cf.src1), cf.k0, cf.k1};
      if (!tgk::gemm_cat_epi_cfg(e, gc, c, ga, blocks))
        throw Error(TG_INTERNAL, "GEMM epilogue: concatenation operands not aligned for the direct-to-LDS kernel");
    } else if (!tgk::gemm_epi_cfg(e, c, ga, blocks)) {
      throw Error(TG_INTERNAL, "GEMM epilogue: no direct-to-LDS launch");
    }
    c.N = d.N;
    c.h_in = h_in;
    c.store_c = store_c;
    if (cs_op >= 0) {
      if (tgk::gemm_epi_colsum_rows(c, ga) != colsum_part_.at(cs_op).rows)
        throw Error(TG_INTERNAL, "GEMM epilogue: column partial rows differ from the plan");
      c.colsum_out = cs_out;
      ga.colsum = reinterpret_cast<double*>(partials_ + cs_off);
    }
    tgk::JitKernel jk = tgk::gemm_epi_kernel(p, fused_code_.data() + code_off, c);
    const size_t js = jit_slots_.size();
    jit_slots_.emplace_back();
    JitSlot& sl = jit_slots_.back();
    sl.name = jk.name;
    sl.grid = blocks;
    sl.gemm = true;
    sl.threads = c.nt;
    sl.gargs = ga;
    for (int k = 0; k < p.n_in; ++k) sl.args.in[k] = p.in[k];
    for (int k = 0; k < p.n_out; ++k) sl.args.out[k] = p.out[k];
    sl.args.seed = p.seed;
    jit_pending_.push_back(std::move(jk));
    return [this, js](hipStream_t st) { launch_jit(js, st); };
  };
  add_node(std::move(n));
}

void Runtime::match_gemm_sums() {
  sum_absorbed_.assign(ops_.size(), 0);
  gemm_sums_.clear();
  if (!use_gemm_sum_ || !use_gemm_group_) return;
  auto pinned = [&](int t) {
    for (int o : outputs_) if (root(o) == root(t)) return true;
    for (auto& c : captures_) if (root(c.second) == root(t)) return true;
    for (auto& w : copy_writebacks_) if (root(w.first) == root(t)) return true;
    return false;
  };
  // The matmul whose product operand t of add op `reader` is: a plain f32 GEMM (no pattern,
  // not deferred) reading whole root tensors, whose product only this add reads.
  auto product = [&](int t, int reader) -> int {
    if (view_[t].root != t || T_[t].dt != F32 || pinned(t)) return -1;
    const int m = T_[t].src;
    if (m < 0 || kinds_[m] != "matmul" || virtual_[m] || attn_of_[m] >= 0 || defer_gemm_[m] || mul_absorbed_[m] ||
        sum_absorbed_[m])
      return -1;
    if (consumers_[t].size() != 1 || consumers_[t][0] != reader) return -1;
    const int a = fld(m, "a"), b = fld(m, "b");
    if (kinds_[T_[view_[a].root].src] == "one_hot" || kinds_[T_[view_[b].root].src] == "one_hot") return -1;
    return m;
  };
  // From the last op back, so a chain's final add claims its inner adds first.
  for (int i = (int)ops_.size() - 1; i >= 0; --i) {
    if (kinds_[i] != "add" || virtual_[i] || sum_absorbed_[i]) continue;
    const int out = O(i).at("out").i32();
    if (view_[out].root != out || !view_[out].contiguous() || T_[out].dt != F32) continue;
    std::vector<int> terms, inner;
    bool ok = true;
    for (int cur = i;;) {
      const int a = fld(cur, "a"), b = fld(cur, "b");
      const int pb = product(b, cur);
      if (pb < 0) { ok = false; break; }
      terms.insert(terms.begin(), pb);
      const int pa = product(a, cur);
      if (pa >= 0) { terms.insert(terms.begin(), pa); break; }
      const int ia = T_[a].src;
      if (view_[a].root != a || ia < 0 || kinds_[ia] != "add" || virtual_[ia] || sum_absorbed_[ia] ||
          consumers_[a].size() != 1 || pinned(a) || (int)terms.size() >= tgk::gd::kMaxSeg) {
        ok = false;
        break;
      }
      inner.push_back(ia);
      cur = ia;
    }
    if (!ok || terms.size() < 2 || terms.size() > (size_t)tgk::gd::kMaxSeg) continue;
    std::vector<tgk::GemmDesc> ds;
    for (int m : terms) {
      tgk::GemmDesc d{};
      const int po = O(m).at("out").i32();
      if (!gemm_desc(m, d) || T_[po].shape != T_[out].shape || d.sCn != 1 || d.sCm != d.N) { ok = false; break; }
      // operands are whole tensors (arena blocks are 256-byte aligned)
      const int a = fld(m, "a"), b = fld(m, "b");
      if (T_[view_[a].root].numel != T_[a].numel || T_[view_[b].root].numel != T_[b].numel) { ok = false; break; }
      d.A = reinterpret_cast<const float*>(uintptr_t(256));
      d.B = reinterpret_cast<const float*>(uintptr_t(256));
      ds.push_back(d);
    }
    if (!ok || !tgk::gemm_sum_ok(ds.data(), (int)ds.size())) continue;
    gemm_sums_[i] = terms;
    sum_absorbed_[i] = 1;
    for (int m : terms) sum_absorbed_[m] = 1;
    for (int a : inner) sum_absorbed_[a] = 1;
  }
}

void Runtime::lower_gemm_sum(int add_op) {
  const std::vector<int> terms = gemm_sums_.at(add_op);
  const int out = O(add_op).at("out").i32();
  Node n;
  n.kind = "gemm";
  n.op = add_op;
  n.detail = "gemm_sum";
  std::vector<tgk::GemmDesc> ds;
  std::vector<int> as, bs;
  double fl = 0, by = 4.0 * T_[out].numel;
  for (int m : terms) {
    tgk::GemmDesc d{};
    if (!gemm_desc(m, d)) throw Error(TG_INTERNAL, "gemm_sum: operand view not expressible");
    const int a = fld(m, "a"), b = fld(m, "b");
    n.reads.push_back(root(a));
    n.reads.push_back(root(b));
    as.push_back(a);
    bs.push_back(b);
    ds.push_back(d);
    fl += 2.0 * (double)d.M * d.N * d.K;
    by += 4.0 * ((double)T_[a].numel + T_[b].numel);
  }
  n.writes.push_back(root(out));
  n.flops = fl;
  n.bytes = by;
  n.shape = shape_str(T_[out].shape) + " sum of " + std::to_string(terms.size()) + " products";
  n.bind = [this, ds, as, bs, out]() -> std::function<void(hipStream_t)> {
    std::vector<tgk::GemmDesc> dd = ds;
    for (size_t s = 0; s < dd.size(); ++s) {
      // every segment's reads and the sum's writes lie inside their tensors
      check_gemm_spans(dd[s], as[s], bs[s], out);
      dd[s].A = (const float*)dptr(as[s]);
      dd[s].B = (const float*)dptr(bs[s]);
      dd[s].C = (float*)dptr(out);
    }
    if (!plan_only_ && !tgk::gemm_sum_ok(dd.data(), (int)dd.size()))
      throw Error(TG_INTERNAL, "gemm_sum: operands not aligned for the direct-to-LDS kernel");
    return [dd](hipStream_t st) { tgk::gemm_sum(dd.data(), (int)dd.size(), st); };
  };
  add_node(std::move(n));
}

void Runtime::emit_gemm_group(const std::vector<DeferredGemm>& grp) {
  const int kind = grp.front().kind;
  Node n;
  n.kind = "gemm";
  n.op = grp.front().op;
  n.detail = "gemm_group";
  double fl = 0, by = 0;
  for (const DeferredGemm& g : grp) {
    n.reads.push_back(root(g.a));
    n.reads.push_back(root(g.b));
    n.writes.push_back(root(g.out));
    fl += 2.0 * (double)g.d.M * g.d.N * g.d.K * g.d.batch;
    by += 4.0 * ((double)T_[g.a].numel + T_[g.b].numel + T_[g.out].numel);
  }
  n.flops = fl;
  n.bytes = by;
  n.shape = "group of " + std::to_string(grp.size()) + " GEMMs";
  n.bind = [this, grp, kind]() -> std::function<void(hipStream_t)> {
    std::vector<tgk::GemmDesc> ds;
    for (const DeferredGemm& g : grp) {
      check_gemm_spans(g.d, g.a, g.b, g.out);
      tgk::GemmDesc d = g.d;
      d.A = (const float*)dptr(g.a);
      d.B = (const float*)dptr(g.b);
      d.C = (float*)dptr(g.out);
      ds.push_back(d);
    }
    std::vector<unsigned char> img;
    int64_t blocks = 0;
    int tiling = 0;
    const size_t off = tgk::gemm_group_table(ds.data(), (int)ds.size(), img, blocks, tiling);
    if (plan_only_) return [](hipStream_t) {};
    void* dev = nullptr;
    hip_check(hipMalloc(&dev, img.size()), "hipMalloc(gemm group table)");
    dev_tables_.push_back(dev);
    hip_check(hipMemcpy(dev, img.data(), img.size(), hipMemcpyHostToDevice), "hipMemcpy(gemm group table)");
    const int np = (int)ds.size();
    return [=](hipStream_t st) { tgk::gemm_group(dev, off, np, blocks, kind, tiling, st); };
  };
  add_node(std::move(n));
}

void Runtime::flush_deferred_gemms() {
  for (int kind = 0; kind < 4; ++kind) {
    std::vector<DeferredGemm> grp;
    for (const DeferredGemm& g : deferred_gemms_)
      if (g.kind == kind) grp.push_back(g);
    if (!grp.empty()) emit_gemm_group(grp);
  }
  deferred_gemms_.clear();
}

// A GEMM that is its own launch (no pattern, not deferred); used to collect independent
// GEMMs into one grouped launch.
bool Runtime::plain_gemm(int j) const {
  if ((kinds_[j] != "matmul" && kinds_[j] != "matmul_batched") || virtual_[j] || is_leaf(j)) return false;
  if (attn_of_[j] >= 0 || group_of_[j] >= 0 || defer_gemm_[j] || gemm_done_[j] || mul_absorbed_[j] || sum_absorbed_[j])
    return false;
  const int a = fld(j, "a"), b = fld(j, "b");
  if (kinds_[T_[view_[a].root].src] == "one_hot" || kinds_[T_[view_[b].root].src] == "one_hot") return false;
  return true;
}

// Tensor t's data exists already: its root is an input / parameter / state, or a node
// emitted so far writes it.
static bool const_kind(const std::string& k) { return k == "const_scalar" || k == "const_fill" || k == "arange"; }
static bool pointwise_const_safe(const std::string& k) {
  return k != "randn" && k != "dropout" && k != "categorical_last" && k != "param_input" && k != "tensor_input" &&
         k != "state_input" && k.rfind("adam_", 0) != 0 && k != "matmul" && k != "matmul_batched";
}

bool Runtime::const_early_ok(int t, int depth) const {
  if (depth > 16) return false;
  if (ready_now(t)) return true;
  const int p = T_[root(t)].src;
  if (p < 0 || is_leaf(p) || virtual_[p] || attn_of_[p] >= 0 || mul_absorbed_[p] || sum_absorbed_[p] ||
      colsum_.count(p) || !pointwise_const_safe(kinds_[p]))
    return false;
  const int g = group_of_[p];
  auto op_ok = [&](int q) {
    if (const_kind(kinds_[q])) return true;
    if (!pointwise_const_safe(kinds_[q]) || is_leaf(q)) return false;
    for (int in : op_inputs(*ops_[q])) {
      const int ip = T_[root(in)].src;
      if (g >= 0 && ip >= 0 && group_of_[ip] == g) continue;   // computed inside the group
      if (!const_early_ok(in, depth + 1)) return false;
    }
    return true;
  };
  if (g < 0) return !gemm_done_[p] && op_ok(p);
  if (group_done_[g] || !groups_[g].dups.empty()) return false;
  for (int q : groups_[g].ops)
    if (!op_ok(q)) return false;
  return true;
}

void Runtime::lower_const_early(int t) {
  if (ready_now(t)) return;
  const int p = T_[root(t)].src;
  const int g = group_of_[p];
  const std::vector<int> ops = g < 0 ? std::vector<int>{p} : groups_[g].ops;
  for (int q : ops)
    if (!const_kind(kinds_[q]))
      for (int in : op_inputs(*ops_[q])) {
        const int ip = T_[root(in)].src;
        if (g >= 0 && ip >= 0 && group_of_[ip] == g) continue;   // computed inside the group
        lower_const_early(in);
      }
  if (g < 0) {
    lower_op(p);
    gemm_done_[p] = 1;
  } else {
    lower_group(g);
    group_done_[g] = 1;
  }
}

bool Runtime::ready_now(int t) const {
  const int r = root(t);
  const int p = T_[r].src;
  if (p < 0 || is_leaf(p)) return true;
  for (const Node& n : nodes_)
    for (int w : n.writes)
      if (w == r) return true;
  return false;
}

void Runtime::lower_op(int i) {
  const std::string& k = kinds_[i];
  const tgj::Value& op = O(i);
  const int out = op.at("out").i32();
  const TInfo& to = T_[out];
  Node n;
  n.kind = k;
  n.op = i;
  n.writes.push_back(root(out));
  n.shape = shape_str(to.shape);
  auto rd = [&](int t) { n.reads.push_back(root(t)); };

  // Broadcast strides of operand view `t` against output dims (right-aligned; size-1 axes
  // of the operand get stride 0).
  auto bstrides = [&](int t, const Dims& od) {
    const View& v = view_[t];
    Dims s(od.size(), 0);
    int off = (int)od.size() - (int)v.dims.size();
    for (size_t d = 0; d < v.dims.size(); ++d) s[off + d] = v.dims[d] == 1 ? 0 : v.strides[d];
    return s;
  };
  auto make_strided = [&](const Dims& od, const Dims& a, const Dims& b, const Dims& c) {
    tgk::Strided sp{};
    // Drop size-1 output dims and merge dims that are contiguous in every operand.
    Dims dd, s0, s1, s2;
    for (size_t d = 0; d < od.size(); ++d) {
      if (od[d] == 1) continue;
      int64_t x = a.empty() ? 0 : a[d], y = b.empty() ? 0 : b[d], z = c.empty() ? 0 : c[d];
      if (!dd.empty() && s0.back() == x * od[d] && s1.back() == y * od[d] && s2.back() == z * od[d]) {
        dd.back() *= od[d]; s0.back() = x; s1.back() = y; s2.back() = z;
      } else {
        dd.push_back(od[d]); s0.push_back(x); s1.push_back(y); s2.push_back(z);
      }
    }
    if (dd.size() > (size_t)tgk::kMaxRank) throw Error(TG_INTERNAL, "rank too large for strided kernel");
    sp.rank = (int)dd.size();
    for (size_t d = 0; d < dd.size(); ++d) { sp.dims[d] = dd[d]; sp.s0[d] = s0[d]; sp.s1[d] = s1[d]; sp.s2[d] = s2[d]; }
    return sp;
  };
  auto need_contig = [&](int t) {
    if (!view_[t].contiguous()) throw Error(TG_INTERNAL, "op '" + k + "' needs a contiguous operand #" + std::to_string(t));
  };

  static const std::map<std::string, int> binops = {{"add", tgk::B_ADD}, {"sub", tgk::B_SUB}, {"mul", tgk::B_MUL},
                                                    {"div", tgk::B_DIV}, {"min", tgk::B_MIN}, {"max", tgk::B_MAX},
                                                    {"less", tgk::B_LESS}, {"greater", tgk::B_GREATER}};
  static const std::map<std::string, int> unops = {
      {"sqrt", tgk::U_SQRT}, {"rsqrt", tgk::U_RSQRT}, {"log", tgk::U_LOG}, {"exp", tgk::U_EXP},
      {"relu", tgk::U_RELU}, {"neg", tgk::U_NEG}, {"abs", tgk::U_ABS}, {"tanh", tgk::U_TANH},
      {"sigmoid", tgk::U_SIGMOID}, {"erf", tgk::U_ERF}, {"sin", tgk::U_SIN}, {"cos", tgk::U_COS}};

  if (binops.count(k)) {
    int a = op.at("a").i32(), b = op.at("b").i32();
    rd(a); rd(b);
    int bop = binops.at(k);
    n.bytes = 4.0 * (T_[a].numel + T_[b].numel + to.numel);
    n.kind = "elementwise";
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      tgk::Strided sp = make_strided(to.shape, bstrides(a, to.shape), bstrides(b, to.shape), {});
      check_span("binary a", T_[root(a)].numel, 0, sp.dims, sp.s0, sp.rank);
      check_span("binary b", T_[root(b)].numel, 0, sp.dims, sp.s1, sp.rank);
      const void* pa = dptr(a); const void* pb = dptr(b); void* po = dptr(out);
      int adt = kdt(T_[a].dt), bdt = kdt(T_[b].dt), odt = kdt(to.dt);
      int64_t cnt = to.numel;
      return [=](hipStream_t st) { tgk::binary(bop, pa, adt, pb, bdt, po, odt, sp, cnt, st); };
    };
  } else if (k == "mul_scalar" || k == "add_scalar") {
    int a = op.at("a").i32();
    need_contig(a); rd(a);
    bool mul = k == "mul_scalar";
    double s = op.at("scalar").num();
    n.bytes = 8.0 * to.numel;
    n.kind = "elementwise";
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      const void* pa = dptr(a); float* po = (float*)dptr(out); int adt = kdt(T_[a].dt); int64_t cnt = to.numel;
      return [=](hipStream_t st) { tgk::scalar_op(mul, pa, adt, s, po, cnt, st); };
    };
  } else if (unops.count(k)) {
    int a = op.at("a").i32();
    need_contig(a); rd(a);
    int uop = unops.at(k);
    n.bytes = 8.0 * to.numel;
    n.kind = "elementwise";
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      const float* pa = (const float*)dptr(a); float* po = (float*)dptr(out); int64_t cnt = to.numel;
      return [=](hipStream_t st) { tgk::unary(uop, pa, po, cnt, st); };
    };
  } else if (k == "relu_grad") {
    int x = op.at("x").i32(), dy = op.at("dy").i32();
    need_contig(x); need_contig(dy); rd(x); rd(dy);
    n.bytes = 12.0 * to.numel;
    n.kind = "elementwise";
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      const float* px = (const float*)dptr(x); const float* pd = (const float*)dptr(dy); float* po = (float*)dptr(out);
      int64_t cnt = to.numel;
      return [=](hipStream_t st) { tgk::relu_grad(px, pd, po, cnt, st); };
    };
  } else if (k == "where") {
    int c = op.at("cond").i32(), a = op.at("a").i32(), b = op.at("b").i32();
    rd(c); rd(a); rd(b);
    n.bytes = 4.0 * (T_[c].numel + T_[a].numel + T_[b].numel + to.numel);
    n.kind = "elementwise";
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      tgk::Strided sp = make_strided(to.shape, bstrides(c, to.shape), bstrides(a, to.shape), bstrides(b, to.shape));
      check_span("where cond", T_[root(c)].numel, 0, sp.dims, sp.s0, sp.rank);
      check_span("where a", T_[root(a)].numel, 0, sp.dims, sp.s1, sp.rank);
      check_span("where b", T_[root(b)].numel, 0, sp.dims, sp.s2, sp.rank);
      const int32_t* pc = (const int32_t*)dptr(c); const void* pa = dptr(a); const void* pb = dptr(b);
      void* po = dptr(out); int dt = kdt(to.dt); int64_t cnt = to.numel;
      return [=](hipStream_t st) { tgk::where(pc, pa, pb, dt, po, sp, cnt, st); };
    };
  } else if (k == "where_causal") {
    int a = op.at("a").i32();
    need_contig(a); rd(a);
    double fill = op.at("fillValue").num();
    int64_t D = to.shape.back(), outer = to.numel / (D * D);
    n.bytes = 8.0 * to.numel;
    n.kind = "elementwise";
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      const float* pa = (const float*)dptr(a); float* po = (float*)dptr(out);
      return [=](hipStream_t st) { tgk::where_causal(pa, po, outer, D, fill, st); };
    };
  } else if (k == "const_scalar" || k == "const_fill") {
    double v = op.at("value").num();
    n.bytes = 4.0 * to.numel;
    n.kind = "fill";
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      void* po = dptr(out); int dt = kdt(to.dt); int64_t cnt = to.numel;
      return [=](hipStream_t st) { tgk::fill(po, dt, v, cnt, st); };
    };
  } else if (k == "arange") {
    n.bytes = 4.0 * to.numel;
    n.kind = "fill";
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      void* po = dptr(out); int dt = kdt(to.dt); int64_t cnt = to.numel;
      return [=](hipStream_t st) { tgk::arange(po, dt, cnt, st); };
    };
  } else if (k == "one_hot") {
    int idx = op.at("indices").i32();
    need_contig(idx); rd(idx);
    int64_t depth = op.at("depth").i64();
    n.bytes = 4.0 * (T_[idx].numel + to.numel);
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      const int32_t* pi = (const int32_t*)dptr(idx); void* po = dptr(out); int dt = kdt(to.dt);
      int64_t rows = T_[idx].numel;
      return [=](hipStream_t st) { tgk::one_hot(pi, rows, depth, po, dt, st); };
    };
  } else if (k == "dropout" || k == "randn" || k == "categorical_last") {
    int seed = op.at("seed").i32();
    rd(seed);
    int64_t salt = op.at("salt").i64();
    uint32_t sc = (uint32_t)(uint64_t)std::fmod((double)salt * 2654435761.0, 4294967296.0);
    if (k == "dropout") {
      int a = op.at("a").i32();
      need_contig(a); rd(a);
      double p = op.at("p").num();
      n.bytes = 8.0 * to.numel;
      n.kind = "elementwise";
      n.bind = [=]() -> std::function<void(hipStream_t)> {
        const float* pa = (const float*)dptr(a); float* po = (float*)dptr(out); const int32_t* ps = (const int32_t*)dptr(seed);
        int64_t cnt = to.numel;
        return [=](hipStream_t st) { tgk::dropout(pa, po, cnt, ps, sc, p, st); };
      };
    } else if (k == "randn") {
      n.bytes = 4.0 * to.numel;
      n.bind = [=]() -> std::function<void(hipStream_t)> {
        float* po = (float*)dptr(out); const int32_t* ps = (const int32_t*)dptr(seed); int64_t cnt = to.numel;
        return [=](hipStream_t st) { tgk::randn(po, cnt, ps, sc, st); };
      };
    } else {
      int a = op.at("a").i32();
      need_contig(a); rd(a);
      int64_t D = T_[a].shape.back(), outer = T_[a].numel / D;
      n.bytes = 4.0 * (T_[a].numel + to.numel);
      n.bind = [=]() -> std::function<void(hipStream_t)> {
        const float* pa = (const float*)dptr(a); int32_t* po = (int32_t*)dptr(out); const int32_t* ps = (const int32_t*)dptr(seed);
        return [=](hipStream_t st) { tgk::categorical(pa, po, outer, D, ps, sc, st); };
      };
    }
  } else if (k == "mean_last" || k == "sum_last" || k == "argmax_last" || k == "log_softmax_last" ||
             k == "softmax_causal_last") {
    int a = op.at("a").i32();
    need_contig(a); rd(a);
    if (T_[a].shape.empty()) throw Error(TG_INVALID_ARGUMENT, k + ": rank-0 input");
    int64_t D = T_[a].shape.back(), outer = D > 0 ? T_[a].numel / D : 0;
    if (k == "softmax_causal_last" && (T_[a].shape.size() < 2 || T_[a].shape[T_[a].shape.size() - 2] != D))
      throw Error(TG_INVALID_ARGUMENT, "softmax_causal_last: last two axes must be square");
    int64_t expect_out = (k == "log_softmax_last" || k == "softmax_causal_last") ? T_[a].numel : outer;
    if (to.numel != expect_out) throw Error(TG_INVALID_ARGUMENT, k + ": output size mismatch");
    n.bytes = 4.0 * (T_[a].numel + to.numel);
    n.kind = (k == "log_softmax_last" || k == "softmax_causal_last") ? "softmax" : "reduce";
    tgk::Strided cells{}, red{};
    cells.rank = 1; cells.dims[0] = outer; cells.s0[0] = D;
    red.rank = 1; red.dims[0] = D; red.s0[0] = 1;
    int64_t cbase = 0;
    if (k == "mean_last" || k == "sum_last") {
      workspace_bytes_ = std::max(workspace_bytes_, (size_t)tgk::sum_workspace_doubles(cells, red, outer, D) * 8);
      cbase = take_counters(tgk::sum_counters(cells, red, outer, D));
      n.ws = true;
    }
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      const float* pa = (const float*)dptr(a); void* po = dptr(out);
      if (k == "mean_last" || k == "sum_last") {
        double div = k == "mean_last" ? (double)D : 1.0;
        double* w = (double*)cur_ws_;
        unsigned* cn = cur_counters_ + cbase;
        return [=](hipStream_t st) { tgk::reduce_sum(pa, (float*)po, cells, red, outer, D, div, w, cn, st); };
      }
      if (k == "argmax_last") return [=](hipStream_t st) { tgk::row_argmax(pa, (int32_t*)po, outer, D, st); };
      if (k == "log_softmax_last") return [=](hipStream_t st) { tgk::log_softmax(pa, (float*)po, outer, D, st); };
      int64_t mats = outer / D;
      return [=](hipStream_t st) { tgk::softmax_causal(pa, (float*)po, mats, D, st); };
    };
  } else if (k == "permute" || k == "reshape" || k == "stop_gradient") {
    // Materialise a strided view (a permute a consumer needs contiguous, or a reshape of
    // a non-contiguous view).
    int a = op.at("a").i32();
    rd(a);
    n.bytes = 8.0 * to.numel;
    n.kind = "copy";
    View src = view_[a];
    if (k == "permute") {
      std::vector<int64_t> perm;
      for (const auto& p : op.at("perm").items) perm.push_back(p.i64());
      View v{src.root, {}, {}};
      for (size_t d = 0; d < perm.size(); ++d) { v.dims.push_back(src.dims[perm[d]]); v.strides.push_back(src.strides[perm[d]]); }
      src = v;
    }
    // reshape of a non-contiguous view: iterate the source view in its own order.
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      tgk::Strided sp = make_strided(src.dims, contiguous_strides(src.dims), src.strides, {});
      check_span("copy dst", T_[root(out)].numel, 0, sp.dims, sp.s0, sp.rank);
      check_span("copy src", T_[src.root].numel, 0, sp.dims, sp.s1, sp.rank);
      void* po = dptr(out); const void* pa = ptr_[src.root]; int64_t cnt = to.numel;
      return [=](hipStream_t st) { tgk::strided_copy(po, pa, sp, cnt, st); };
    };
  } else if (k == "broadcast_to") {
    int a = op.at("a").i32();
    rd(a);
    n.bytes = 4.0 * (T_[a].numel + to.numel);
    n.kind = "copy";
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      tgk::Strided sp = make_strided(to.shape, contiguous_strides(to.shape), bstrides(a, to.shape), {});
      check_span("broadcast src", T_[root(a)].numel, 0, sp.dims, sp.s1, sp.rank);
      void* po = dptr(out); const void* pa = dptr(a); int64_t cnt = to.numel;
      return [=](hipStream_t st) { tgk::strided_copy(po, pa, sp, cnt, st); };
    };
  } else if (k == "slice_range" || k == "scatter_axis" || k == "concat") {
    n.kind = "copy";
    int64_t ax = op.at("axis").i64();
    std::vector<int> ins;
    if (k == "concat") for (const auto& x : op.at("inputs").items) ins.push_back(x.i32());
    else ins.push_back(op.at("a").i32());
    for (int t : ins) { need_contig(t); rd(t); }
    int64_t total_in = 0;
    for (int t : ins) total_in += T_[t].numel;
    n.bytes = 4.0 * (total_in + to.numel);
    int64_t start = k == "concat" ? 0 : op.at("start").i64();
    // along the last axis: one launch writing the output rows in order
    if (k == "concat" && ax == (int64_t)to.shape.size() - 1 && (int)ins.size() <= tgk::kConcatMax &&
        to.numel < (int64_t(1) << 31)) {
      n.bind = [=]() -> std::function<void(hipStream_t)> {
        tgk::ConcatLast c{};
        c.n = (int)ins.size();
        int64_t w = 0;
        const int64_t rows = to.shape.empty() || to.shape.back() == 0 ? 0 : to.numel / to.shape.back();
        for (int i = 0; i < c.n; ++i) {
          const Dims& is = T_[ins[i]].shape;
          if (T_[root(ins[i])].numel < T_[ins[i]].numel || T_[ins[i]].numel != rows * is.back())
            throw Error(TG_INTERNAL, "concat: input smaller than its shape");
          c.src[i] = (const uint32_t*)dptr(ins[i]);
          c.off[i] = (uint32_t)w;
          w += is.back();
        }
        c.off[c.n] = (uint32_t)w;
        if (w != to.shape.back() || T_[root(out)].numel < to.numel) throw Error(TG_INTERNAL, "concat: widths do not add up");
        uint32_t* po = (uint32_t*)dptr(out);
        return [=](hipStream_t st) { tgk::concat_last(po, c, rows, st); };
      };
      add_node(std::move(n));
      return;
    }
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      std::vector<std::function<void(hipStream_t)>> parts;
      Dims os = contiguous_strides(to.shape);
      if (k == "scatter_axis") {
        void* po = dptr(out); int64_t cnt = to.numel;
        parts.push_back([=](hipStream_t st) { tgk::fill(po, tgk::DT_F32, 0.0, cnt, st); });
      }
      int64_t off = 0;
      for (int t : ins) {
        const Dims& is = T_[t].shape;
        Dims src_str = contiguous_strides(is);
        if (k == "slice_range") {
          // out[..., j, ...] = a[..., j + start, ...]
          Dims s1 = src_str;
          int64_t base = start * src_str[ax];
          tgk::Strided sp = make_strided(to.shape, os, s1, {});
          check_span("slice dst", T_[root(out)].numel, 0, sp.dims, sp.s0, sp.rank);
          check_span("slice src", T_[root(t)].numel, base, sp.dims, sp.s1, sp.rank);
          void* po = dptr(out); const float* pa = (const float*)dptr(t) + base; int64_t cnt = to.numel;
          parts.push_back([=](hipStream_t st) { tgk::strided_copy(po, pa, sp, cnt, st); });
        } else {
          // out[..., j + offset, ...] = a[..., j, ...]
          int64_t base = (k == "concat" ? off : start) * os[ax];
          tgk::Strided sp = make_strided(is, os, src_str, {});
          check_span("concat dst", T_[root(out)].numel, base, sp.dims, sp.s0, sp.rank);
          check_span("concat src", T_[root(t)].numel, 0, sp.dims, sp.s1, sp.rank);
          float* po = (float*)dptr(out) + base; const void* pa = dptr(t); int64_t cnt = T_[t].numel;
          parts.push_back([=](hipStream_t st) { tgk::strided_copy(po, pa, sp, cnt, st); });
          off += is[ax];
        }
      }
      return [=](hipStream_t st) { for (auto& f : parts) f(st); };
    };
  } else if (k == "sum_to_shape") {
    int a = op.at("a").i32();
    need_contig(a); rd(a);
    const Dims& as = T_[a].shape;
    n.bytes = 4.0 * (T_[a].numel + to.numel);
    n.kind = "reduce";
    Dims ast = contiguous_strides(as);
    int rdiff = (int)as.size() - (int)to.shape.size();
    Dims cd, cs, rdd, rs;
    for (int d = 0; d < (int)as.size(); ++d) {
      bool reduced = d < rdiff || (to.shape[d - rdiff] == 1 && as[d] != 1);
      if (as[d] == 1) continue;
      if (reduced) { rdd.push_back(as[d]); rs.push_back(ast[d]); }
      else { cd.push_back(as[d]); cs.push_back(ast[d]); }
    }
    tgk::Strided cells = make_strided(cd, cs, {}, {});
    tgk::Strided red = make_strided(rdd, rs, {}, {});
    int64_t ncells = prod(cd), nred = prod(rdd);
    if (ncells != to.numel) throw Error(TG_INTERNAL, "sum_to_shape: cell count mismatch");
    // [B, C, L] form (kept axis in the middle of a contiguous array), read only by the
    // optimizer: joins the deferred column-sum launch
    if (use_gemm_group_ && use_colsum_mid_ && any_deferred_colsum_ && (int)deferred_midsum_.size() < tgk::kMidSumMax &&
        cells.rank == 1 && red.rank == 2 && red.s0[1] == 1 && cells.s0[0] == red.dims[1] &&
        red.s0[0] == cells.dims[0] * cells.s0[0] && view_[a].root == a && view_[a].contiguous() &&
        view_[out].root == out && view_[out].contiguous() && only_optimizer_reads(out)) {
      deferred_midsum_.push_back({a, out, red.dims[0], cells.dims[0], red.dims[1]});
      return;
    }
    workspace_bytes_ = std::max(workspace_bytes_, (size_t)tgk::sum_workspace_doubles(cells, red, ncells, nred) * 8);
    const int64_t cbase = take_counters(tgk::sum_counters(cells, red, ncells, nred));
    n.ws = true;
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      {
        int64_t dd[2 * tgk::kMaxRank], ss[2 * tgk::kMaxRank];
        int r = 0;
        for (int q = 0; q < cells.rank; ++q) { dd[r] = cells.dims[q]; ss[r++] = cells.s0[q]; }
        for (int q = 0; q < red.rank; ++q) { dd[r] = red.dims[q]; ss[r++] = red.s0[q]; }
        check_span("sum_to_shape src", T_[root(a)].numel, 0, dd, ss, r);
      }
      const float* pa = (const float*)dptr(a); float* po = (float*)dptr(out);
      double* w = (double*)cur_ws_;
      unsigned* cn = cur_counters_ + cbase;
      return [=](hipStream_t st) { tgk::reduce_sum(pa, po, cells, red, ncells, nred, 1.0, w, cn, st); };
    };
  } else if (k == "matmul" || k == "matmul_batched") {
    int a = op.at("a").i32(), b = op.at("b").i32();
    bool batched = k == "matmul_batched";
    const Dims& ash = T_[a].shape;
    const Dims& bsh = T_[b].shape;
    int64_t M = ash[ash.size() - 2], K = ash.back(), N = to.shape.back();
    int64_t batch = T_[a].numel / (M * K);
    n.flops = 2.0 * (double)batch * M * N * K;
    n.kind = "gemm";
    n.shape = shape_str(ash) + "x" + shape_str(bsh);
    if (N != bsh.back()) n.shape += " first " + std::to_string(N) + " columns";
    // Pattern: embedding forward, one_hot(idx) @ table.
    int asrc = T_[view_[a].root].src;
    // The one-hot must be read as laid out ([rows, depth] row-major, rows = batch * M,
    // depth = K), not transposed; with depth 1 a transpose is also contiguous.
    if (!batched && asrc >= 0 && kinds_[asrc] == "one_hot" && view_[a].contiguous() && view_[b].contiguous() &&
        T_[view_[a].root].dt == F32 && T_[fld(asrc, "indices")].numel == batch * M &&
        O(asrc).at("depth").i64() == K) {
      int idx = fld(asrc, "indices");
      rd(idx); rd(b);
      n.kind = "gather";
      n.flops = 0;
      int64_t rows = batch * M;
      n.bytes = 4.0 * (rows + rows * N + rows * N);
      n.bind = [=]() -> std::function<void(hipStream_t)> {
        const int32_t* pi = (const int32_t*)dptr(idx); const float* pt = (const float*)dptr(b); float* po = (float*)dptr(out);
        return [=](hipStream_t st) { tgk::gather_rows(pi, rows, pt, K, N, po, st); };
      };
      add_node(std::move(n));
      return;
    }
    // Pattern: embedding gradient, transpose(one_hot(idx)) @ dy.
    if (!batched && asrc >= 0 && kinds_[asrc] == "one_hot" && ash.size() == 2 && T_[view_[a].root].dt == F32) {
      const View& va = view_[a];
      int64_t rows = T_[fld(asrc, "indices")].numel, V = O(asrc).at("depth").i64();
      if (va.dims.size() == 2 && va.dims[0] == V && va.dims[1] == rows && va.strides[0] == 1 && va.strides[1] == V &&
          view_[b].contiguous() && V <= 8192) {
        const DeferredScatter sc{i, fld(asrc, "indices"), b, out, rows, V, N, n.shape};
        if (use_gemm_group_ && use_colsum_scatter_ && deferred_scatter_.empty() && tgk::scatter_scan_form(rows, V) &&
            only_optimizer_reads(out)) {
          deferred_scatter_.push_back(sc);
          return;
        }
        emit_scatter(sc);
        return;
      }
    }
    // Pattern: A is the transpose of a last-axis concatenation [R, K0 + K1 + ...] (the
    // weight gradient of a layer fed by a skip concatenation): one GEMM per source, each
    // reading its source in place and writing its own rows of the product, so no tile runs
    // on the concatenation's unaligned rows or straddles two sources.
    std::vector<int> cat_src;
    std::vector<int64_t> cat_off;
    tgk::GemmDesc d{};
    // Pattern: A is a last-axis concatenation of two sources: one GEMM reading both in place.
    if (cat_fwd_.count(i)) {
      const CatFwd cf = cat_fwd_.at(i);
      if (!gemm_desc(i, d)) throw Error(TG_INTERNAL, "gemm: operand view not expressible (" + n.shape + ")");
      d.sAm = cf.k0;   // A0 = the first source, [M, k0] contiguous
      if (gemm_epi_mode_ != kEpiOff && use_jit_) {
        bool store_c = false;
        const int gi = epi_group(i, out, d, store_c, &cf);
        if (gi >= 0 && (gemm_epi_mode_ == kEpiAll || epi_cheap(gi))) {
          lower_gemm_epi(i, d, a, b, out, gi, store_c, &cf);
          return;
        }
      }
      rd(cf.src0); rd(cf.src1); rd(b);
      n.detail = "gemm_cat";
      n.bytes = 4.0 * (T_[a].numel + T_[b].numel + to.numel);
      n.bind = [=]() -> std::function<void(hipStream_t)> {
        check_cat_spans(d, cf, b, out, true);
        tgk::GemmDesc g = d;
        g.A = (const float*)dptr(cf.src0);
        g.B = (const float*)dptr(b);
        g.C = (float*)dptr(out);
        const tgk::GemmCat gc{(const float*)dptr(cf.src1), cf.k0, cf.k1};
        if (!plan_only_ && !tgk::gemm_cat_ok(g, gc))
          throw Error(TG_INTERNAL, "gemm_cat: operands not aligned for the direct-to-LDS kernel");
        return [=](hipStream_t st) { tgk::gemm_cat(g, gc, st); };
      };
      add_node(std::move(n));
      return;
    }
    if (!batched && !defer_gemm_[i] && concat_transposed(a, cat_src, cat_off) && gemm_desc(i, d) && d.batch == 1 &&
        d.sCn == 1 && d.sCm == N && view_[out].root == out && view_[out].contiguous()) {
      std::vector<tgk::GemmDesc> ds;
      int64_t ws = 0;
      for (size_t s = 0; s < cat_src.size(); ++s) {
        tgk::GemmDesc g = d;
        g.M = T_[cat_src[s]].shape.back();
        g.sAm = 1;
        g.sAk = g.M;
        ws = std::max(ws, tgk::gemm_workspace_floats(g));
        ds.push_back(g);
        rd(cat_src[s]);
      }
      rd(b);
      workspace_bytes_ = std::max(workspace_bytes_, (size_t)ws * 4);
      n.ws = ws > 0;
      n.bytes = 4.0 * (T_[a].numel + T_[b].numel + to.numel);
      n.shape += " by " + std::to_string(cat_src.size()) + " sources";
      n.bind = [=]() -> std::function<void(hipStream_t)> {
        std::vector<tgk::GemmDesc> gs = ds;
        for (size_t s = 0; s < gs.size(); ++s) {
          tgk::GemmDesc& g = gs[s];
          const int64_t da[2] = {g.M, g.K}, sa[2] = {g.sAm, g.sAk};
          const int64_t db[2] = {g.K, g.N}, sb[2] = {g.sBk, g.sBn};
          const int64_t dc[2] = {g.M, g.N}, sc[2] = {g.sCm, g.sCn};
          check_span("gemm A (concatenation source)", T_[root(cat_src[s])].numel, 0, da, sa, 2);
          check_span("gemm B", T_[root(b)].numel, 0, db, sb, 2);
          check_span("gemm C (source rows)", T_[root(out)].numel, cat_off[s] * g.sCm, dc, sc, 2);
          g.A = (const float*)dptr(cat_src[s]);
          g.B = (const float*)dptr(b);
          g.C = (float*)dptr(out) + cat_off[s] * g.sCm;
        }
        float* w = cur_ws_;
        return [=](hipStream_t st) { for (const tgk::GemmDesc& g : gs) tgk::gemm(g, w, st); };
      };
      add_node(std::move(n));
      return;
    }
    rd(a); rd(b);
    if (!gemm_desc(i, d)) throw Error(TG_INTERNAL, "gemm: operand view not expressible (" + n.shape + ")");
    int64_t ws = tgk::gemm_workspace_floats(d);
    if (defer_gemm_[i]) {
      deferred_gemms_.push_back({i, d, a, b, out, tgk::gemm_group_kind(d)});
      return;
    }
    if (use_gemm_group_ && tgk::gemm_prefers_group(d)) {
      const int kind = tgk::gemm_group_kind(d);
      std::vector<DeferredGemm> grp{{i, d, a, b, out, kind}};
      for (int j = i + 1; j < (int)ops_.size() && j <= i + 64 && grp.size() < 8; ++j) {
        if (!plain_gemm(j)) continue;
        tgk::GemmDesc dj{};
        if (!gemm_desc(j, dj) || !tgk::gemm_prefers_group(dj) || tgk::gemm_group_kind(dj) != kind) continue;
        const int aj = fld(j, "a"), bj = fld(j, "b");
        if (!ready_now(aj) || !ready_now(bj)) continue;
        grp.push_back({j, dj, aj, bj, O(j).at("out").i32(), kind});
      }
      if (grp.size() > 1) {
        for (const DeferredGemm& g : grp) gemm_done_[g.op] = 1;
        emit_gemm_group(grp);
        return;
      }
    }
    if (gemm_epi_mode_ != kEpiOff && use_jit_) {
      bool store_c = false;
      const int gi = epi_group(i, out, d, store_c);
      if (gi >= 0 && (gemm_epi_mode_ == kEpiAll || epi_cheap(gi))) {
        lower_gemm_epi(i, d, a, b, out, gi, store_c);
        return;
      }
    }
    workspace_bytes_ = std::max(workspace_bytes_, (size_t)ws * 4);
    n.bytes = 4.0 * (T_[a].numel + T_[b].numel + to.numel);
    n.ws = ws > 0;
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      check_gemm_spans(d, a, b, out);
      tgk::GemmDesc g = d;
      g.A = (const float*)dptr(a);
      g.B = (const float*)dptr(b);
      g.C = (float*)dptr(out);
      float* w = cur_ws_;
      return [=](hipStream_t st) { tgk::gemm(g, w, st); };
    };
  } else if (k == "conv2d" || k == "conv2d_input_grad" || k == "conv2d_weight_grad") {
    tgk::ConvDesc c{};
    c.sH = op.at("strideH").i64(); c.sW = op.at("strideW").i64();
    c.pH = op.at("padH").i64(); c.pW = op.at("padW").i64(); c.G = op.at("groups").i64();
    int x = -1, w = -1, dy = -1;
    if (k == "conv2d") { x = op.at("input").i32(); w = op.at("weight").i32(); }
    else if (k == "conv2d_input_grad") { w = op.at("weight").i32(); dy = op.at("dy").i32(); }
    else { x = op.at("input").i32(); dy = op.at("dy").i32(); }
    Dims xs = k == "conv2d_input_grad" ? to.shape : T_[x].shape;
    Dims ws = k == "conv2d_weight_grad" ? to.shape : T_[w].shape;
    Dims ys = k == "conv2d" ? to.shape : T_[dy].shape;
    c.B = xs[0]; c.Cin = xs[1]; c.H = xs[2]; c.W = xs[3];
    c.Cout = ws[0]; c.CinPG = ws[1]; c.kH = ws[2]; c.kW = ws[3];
    c.Ho = ys[2]; c.Wo = ys[3];
    for (int t : {x, w, dy}) if (t >= 0) { need_contig(t); rd(t); }
    if (x >= 0 && T_[x].numel != c.B * c.Cin * c.H * c.W) throw Error(TG_INVALID_ARGUMENT, "conv: input size mismatch");
    if (w >= 0 && T_[w].numel != c.Cout * c.CinPG * c.kH * c.kW) throw Error(TG_INVALID_ARGUMENT, "conv: weight size mismatch");
    if (dy >= 0 && T_[dy].numel != c.B * c.Cout * c.Ho * c.Wo) throw Error(TG_INVALID_ARGUMENT, "conv: dy size mismatch");
    if (to.numel != (k == "conv2d" ? c.B * c.Cout * c.Ho * c.Wo : k == "conv2d_input_grad" ? c.B * c.Cin * c.H * c.W
                                                                  : c.Cout * c.CinPG * c.kH * c.kW))
      throw Error(TG_INVALID_ARGUMENT, "conv: output size mismatch");
    if (c.G <= 0 || c.Cout % c.G != 0 || c.CinPG * c.G != c.Cin) throw Error(TG_INVALID_ARGUMENT, "conv: bad groups");
    n.flops = 2.0 * c.B * c.Cout * c.Ho * c.Wo * c.CinPG * c.kH * c.kW;
    n.bytes = 4.0 * (prod(xs) + prod(ws) + prod(ys));
    n.kind = "conv";
    n.shape = shape_str(xs) + "*" + shape_str(ws);
    // Implicit GEMM on the matrix cores by default; TG_CONV=direct selects the direct f64
    // kernels (bit-exact with the evaluator, far slower).
    const bool mfma = use_conv_gemm_ && tgk::conv_gemm_ok(c);
    if (mfma && k == "conv2d_weight_grad") {
      const int64_t wsb = tgk::conv_gemm_workspace_bytes(c);
      workspace_bytes_ = std::max(workspace_bytes_, (size_t)wsb);
      n.ws = wsb > 0;
    }
    if (!mfma) n.detail = "direct";
    // The output read only by a group of its own applying the layer's pointwise step, done
    // at the store instead (the group is not lowered, its input never stored):
    //  forward: relu(add(y, bias)) with bias [Cout] broadcast over channels (one group);
    //  input gradient: relu_grad(mask, dx) with mask laid out as dx.
    int epi_out = out, ebias = -1, emask = -1;
    auto lone_group = [&](int op) {
      const int g = group_of_[op];
      return g >= 0 && groups_[g].dups.empty() && !group_done_[g] ? g : -1;
    };
    auto plain_out = [&](int t) {
      return view_[t].root == t && view_[t].contiguous() && T_[t].dt == F32 && T_[t].numel == to.numel;
    };
    if (mfma && T_[out].dt == F32 && view_[out].root == out && consumers_[out].size() == 1) {
      const int u = consumers_[out][0];
      if (k == "conv2d" && c.G == 1 && kinds_[u] == "add" && lone_group(u) >= 0 &&
          groups_[lone_group(u)].ops.size() == 2 && groups_[lone_group(u)].ops[0] == u) {
        const int g = lone_group(u);
        const int rl = groups_[g].ops[1];
        const int a_out = O(u).at("out").i32();
        const int bias = fld(u, "a") == out ? fld(u, "b") : fld(u, "a");
        Dims bs = T_[bias].shape;
        while (!bs.empty() && bs.front() == 1) bs.erase(bs.begin());
        if (kinds_[rl] == "relu" && fld(rl, "a") == a_out && consumers_[a_out].size() == 1 && bias != out &&
            T_[bias].dt == F32 && view_[bias].contiguous() && T_[bias].numel == c.Cout &&
            bs == Dims({c.Cout, 1, 1}) && plain_out(O(rl).at("out").i32())) {
          bool pinned_a = false;
          for (int o : outputs_) pinned_a = pinned_a || root(o) == root(a_out);
          for (auto& cp : captures_) pinned_a = pinned_a || root(cp.second) == root(a_out);
          if (!pinned_a) {
            epi_out = O(rl).at("out").i32();
            ebias = bias;
            group_done_[g] = 1;
            n.detail = "conv2d,add,relu";
          }
        }
      } else if (k == "conv2d_input_grad" && kinds_[u] == "relu_grad" && fld(u, "dy") == out && lone_group(u) >= 0 &&
                 groups_[lone_group(u)].ops.size() == 1) {
        const int m = fld(u, "x");
        if (m != out && T_[m].dt == F32 && T_[m].shape == to.shape && view_[m].contiguous() &&
            plain_out(O(u).at("out").i32())) {
          epi_out = O(u).at("out").i32();
          emask = m;
          group_done_[lone_group(u)] = 1;
          n.detail = "conv2d_input_grad,relu_grad";
        }
      }
    }
    if (epi_out != out) {
      n.writes = {root(epi_out)};
      if (ebias >= 0) rd(ebias);
      if (emask >= 0) rd(emask);
    }
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      float* po = (float*)dptr(epi_out);
      if (k == "conv2d") {
        const float* px = (const float*)dptr(x); const float* pw = (const float*)dptr(w);
        const float* pb = ebias >= 0 ? (const float*)dptr(ebias) : nullptr;
        if (mfma) return [=](hipStream_t st) { tgk::conv2d_gemm(px, pw, po, c, st, pb); };
        return [=](hipStream_t st) { tgk::conv2d(px, pw, po, c, st); };
      }
      if (k == "conv2d_input_grad") {
        const float* pw = (const float*)dptr(w); const float* pd = (const float*)dptr(dy);
        const float* pm = emask >= 0 ? (const float*)dptr(emask) : nullptr;
        if (mfma) return [=](hipStream_t st) { tgk::conv2d_input_grad_gemm(pw, pd, po, c, st, pm); };
        return [=](hipStream_t st) { tgk::conv2d_input_grad(pw, pd, po, c, st); };
      }
      const float* px = (const float*)dptr(x); const float* pd = (const float*)dptr(dy);
      if (mfma) {
        float* wk = cur_ws_;
        return [=](hipStream_t st) { tgk::conv2d_weight_grad_gemm(px, pd, po, c, wk, st); };
      }
      return [=](hipStream_t st) { tgk::conv2d_weight_grad(px, pd, po, c, nullptr, st); };
    };
  } else if (k == "max_pool_2d" || k == "max_pool_2d_grad") {
    int x = op.at("input").i32();
    need_contig(x); rd(x);
    int dy = k == "max_pool_2d_grad" ? op.at("dy").i32() : -1;
    if (dy >= 0) { need_contig(dy); rd(dy); }
    tgk::PoolDesc p{};
    const Dims& xs = T_[x].shape;
    Dims ys = dy >= 0 ? T_[dy].shape : to.shape;
    p.B = xs[0]; p.C = xs[1]; p.H = xs[2]; p.W = xs[3]; p.Ho = ys[2]; p.Wo = ys[3];
    p.kH = op.at("kH").i64(); p.kW = op.at("kW").i64(); p.sH = op.at("strideH").i64(); p.sW = op.at("strideW").i64();
    p.pH = op.at("padH").i64(); p.pW = op.at("padW").i64();
    if (dy < 0 && to.numel != p.B * p.C * p.Ho * p.Wo) throw Error(TG_INVALID_ARGUMENT, "pool: output size mismatch");
    if (dy >= 0 && (to.numel != prod(xs) || ys[0] != p.B || ys[1] != p.C)) throw Error(TG_INVALID_ARGUMENT, "pool grad: size mismatch");
    n.bytes = 4.0 * (prod(xs) + prod(ys) + (dy >= 0 ? prod(xs) : 0));
    n.kind = "pool";
    // The gradient read only by relu_grad(x', it) with x' the pool's own input (the ReLU
    // output it pools, after relu_grads_from_outputs), in a group of its own or none: the
    // pool launch applies the mask and writes the relu_grad's output; the op is skipped.
    int rg_out = out;
    if (dy >= 0 && consumers_[out].size() == 1 && T_[out].dt == F32 && view_[out].root == out) {
      const int c = consumers_[out][0];
      const int g = group_of_[c];
      if (kinds_[c] == "relu_grad" && fld(c, "dy") == out && fld(c, "x") != out && root(fld(c, "x")) == root(x) &&
          T_[fld(c, "x")].shape == xs && view_[fld(c, "x")].contiguous() && !virtual_[c] &&
          (g < 0 || (groups_[g].ops.size() == 1 && groups_[g].dups.empty() && !group_done_[g]))) {
        const int ro = O(c).at("out").i32();
        if (view_[ro].root == ro && view_[ro].contiguous() && T_[ro].numel == to.numel && T_[ro].dt == F32) {
          rg_out = ro;
          if (g >= 0) group_done_[g] = 1;
          else pool_absorbed_[c] = 1;
          n.writes = {root(ro)};
          n.detail = "max_pool_2d_grad,relu_grad";
        }
      }
    }
    const bool relu = rg_out != out;
    n.bind = [=]() -> std::function<void(hipStream_t)> {
      const float* px = (const float*)dptr(x); float* po = (float*)dptr(rg_out);
      if (dy < 0) return [=](hipStream_t st) { tgk::max_pool(px, po, p, st); };
      const float* pd = (const float*)dptr(dy);
      return [=](hipStream_t st) { tgk::max_pool_grad(px, pd, po, p, st, relu); };
    };
  } else if (k == "adam_update_m" || k == "adam_update_v" || k == "adam_update_p") {
    throw Error(TG_INTERNAL, "adam op outside the fused update");
  } else {
    throw Error(TG_INVALID_ARGUMENT, "IR: unsupported op kind '" + k + "'");
  }
  add_node(std::move(n));
}

// Device memory: persistent roots get dedicated regions; intermediates are pooled by
// liveness over the node order (best fit). Tensor inputs live in one contiguous region
// so a step uploads them with a single copy.
void Runtime::split_init_nodes() {
  init_nodes_.clear();
  init_roots_.clear();
  std::set<int> pinned;
  for (int o : outputs_) pinned.insert(root(o));
  for (auto& c : captures_) pinned.insert(root(c.second));
  for (auto& w : copy_writebacks_) pinned.insert(root(w.first));
  std::vector<Node> step;
  for (auto& n : nodes_) {
    bool inv = n.kind != "adam_multi" && n.kind != "sgd_multi" && n.kind != "grad_norm" && !n.writes.empty();
    for (int r : n.reads) if (!init_roots_.count(r)) inv = false;
    for (int w : n.writes) if (pinned.count(w)) inv = false;
    if (inv) {
      for (int w : n.writes) init_roots_.insert(w);
      init_nodes_.push_back(std::move(n));
    } else {
      step.push_back(std::move(n));
    }
  }
  nodes_ = std::move(step);
}

void Runtime::allocate() {
  const size_t nT = T_.size();
  ptr_.assign(nT, nullptr);
  std::vector<bool> persistent(nT, false), used(nT, false);
  std::set<int> input_roots;
  for (size_t i = 0; i < ops_.size(); ++i) {
    int out = ops_[i]->at("out").i32();
    const std::string& k = kinds_[i];
    if (k == "param_input" || k == "state_input") persistent[out] = true;
    if (k == "tensor_input") input_roots.insert(out);
  }
  for (int o : outputs_) persistent[root(o)] = true;
  for (auto& c : captures_) persistent[root(c.second)] = true;
  for (auto& w : copy_writebacks_) persistent[root(w.first)] = true;
  for (int r : init_roots_) persistent[r] = used[r] = true;

  std::vector<int> def(nT, -1), last(nT, -1);
  for (size_t ni = 0; ni < nodes_.size(); ++ni) {
    for (int r : nodes_[ni].writes) { if (def[r] < 0) def[r] = (int)ni; used[r] = true; }
    for (int r : nodes_[ni].reads) { last[r] = std::max(last[r], (int)ni); used[r] = true; }
  }
  for (int o : outputs_) used[root(o)] = true;

  // Layout: [persistent params/state/outputs][pooled intermediates]; inputs separately.
  auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
  size_t off = 0;
  std::vector<size_t> offset(nT, 0);
  std::vector<bool> placed(nT, false);
  for (size_t t = 0; t < nT; ++t) {
    if (root((int)t) != (int)t || input_roots.count((int)t)) continue;
    if (persistent[t] && (used[t] || kinds_[T_[t].src] == "param_input" || kinds_[T_[t].src] == "state_input")) {
      if (parent && kinds_[T_[t].src] == "param_input") continue;  // shared with parent
      offset[t] = off; placed[t] = true;
      off = align(off + std::max<int64_t>(4, T_[t].numel * 4));
    }
  }
  // Pool: walk nodes in order; allocate each written intermediate root, free after last read.
  struct Block { size_t off, size; };
  std::vector<Block> free_list;
  size_t pool_base = off, pool_end = off;
  std::vector<std::vector<int>> frees_at(nodes_.size());
  for (size_t t = 0; t < nT; ++t)
    if (!persistent[t] && !input_roots.count((int)t) && root((int)t) == (int)t && used[t] && last[t] >= 0)
      frees_at[last[t]].push_back((int)t);
  std::vector<size_t> block_size(nT, 0);   // size of the pooled block a root occupies
  for (size_t ni = 0; ni < nodes_.size(); ++ni) {
    // Blocks of outputs nothing reads return to the pool only after every output of the
    // node is placed: outputs of one launch must never share memory.
    std::vector<Block> dead;
    for (int r : nodes_[ni].writes) {
      if (persistent[r] || input_roots.count(r) || placed[r]) continue;
      size_t need = align(std::max<int64_t>(4, T_[r].numel * 4));
      int best = -1;
      for (size_t q = 0; q < free_list.size(); ++q)
        if (free_list[q].size >= need && (best < 0 || free_list[q].size < free_list[best].size)) best = (int)q;
      if (best >= 0) {
        offset[r] = free_list[best].off;
        block_size[r] = free_list[best].size;   // best fit never splits a block
        free_list.erase(free_list.begin() + best);
      } else {
        offset[r] = pool_end;
        block_size[r] = need;
        pool_end += need;
      }
      placed[r] = true;
      if (last[r] < 0) dead.push_back({offset[r], block_size[r]});
    }
    free_list.insert(free_list.end(), dead.begin(), dead.end());
    for (int r : frees_at[ni]) free_list.push_back({offset[r], block_size[r]});
  }
  (void)pool_base;
  // Plan-only mode (tg_plan, no device) also proves the layout: no two pooled buffers
  // whose lifetimes (first write .. last read, in node order) meet may overlap, and no
  // buffer is read before it is written.
  if (plan_only_) {
    std::vector<int> pooled;
    for (size_t t = 0; t < nT; ++t)
      if (placed[t] && !persistent[t] && root((int)t) == (int)t && def[t] >= 0) pooled.push_back((int)t);
    for (size_t x = 0; x < pooled.size(); ++x)
      for (size_t y = x + 1; y < pooled.size(); ++y) {
        const int a = pooled[x], b = pooled[y];
        const int la = std::max(last[a], def[a]), lb = std::max(last[b], def[b]);
        if (la < def[b] || lb < def[a]) continue;
        const size_t ea = offset[a] + (size_t)T_[a].numel * 4, eb = offset[b] + (size_t)T_[b].numel * 4;
        if (ea <= offset[b] || eb <= offset[a]) continue;
        throw Error(TG_INTERNAL, "memory plan: tensors " + std::to_string(a) + " and " + std::to_string(b) +
                                     " are live together but overlap");
      }
    for (int t : pooled)
      if (last[t] >= 0 && def[t] > last[t])
        throw Error(TG_INTERNAL, "memory plan: tensor " + std::to_string(t) + " is read before it is written");
  }
  arena_bytes_ = std::max<size_t>(pool_end, 256);
  // Plan-only mode lays out a fake address space so every bind can run its checks.
  char* fake = reinterpret_cast<char*>((uintptr_t)1 << 40);
  if (plan_only_) arena_ = fake;
  else hip_check(hipMalloc(&arena_, arena_bytes_), "hipMalloc(arena)");
  for (size_t t = 0; t < nT; ++t) if (placed[t]) ptr_[t] = arena_ + offset[t];
  if (parent) {
    for (auto& kv : param_root) {
      auto it = parent->param_root.find(kv.first);
      if (it == parent->param_root.end()) throw Error(TG_INVALID_ARGUMENT, "compileForward: parent has no param '" + kv.first + "'");
      if (parent->T_[it->second].numel != T_[kv.second].numel)
        throw Error(TG_INVALID_ARGUMENT, "compileForward: param '" + kv.first + "' size differs from parent");
      ptr_[kv.second] = parent->ptr_[it->second];
    }
  }
  // Inputs: the caller's tensors first, then the runtime's per-step scalars (optimizer
  // scalars, PRNG seed), so a step with device-resident data uploads only the tail.
  auto internal = [&](int t) {
    const std::string& nm = O(T_[t].src).at("name").str();
    if (nm == "__prngSeed") return true;
    if (!opt_cfg_) return false;
    for (const char* f : {"lrtInputName", "decayShrinkInputName", "lrInputName"}) {
      const tgj::Value* v = opt_cfg_->get(f);
      if (v && v->kind == tgj::Value::String && v->str() == nm) return true;
    }
    return false;
  };
  size_t ioff = 0;
  for (int t : input_roots) if (!internal(t)) { input_offset_[t] = ioff; ioff = align(ioff + std::max<int64_t>(4, T_[t].numel * 4)); }
  user_bytes_ = ioff;
  for (int t : input_roots) if (internal(t)) { input_offset_[t] = ioff; ioff = align(ioff + std::max<int64_t>(4, T_[t].numel * 4)); }
  input_region_bytes_ = std::max<size_t>(ioff, 256);
  if (plan_only_) {
    fused_code_dev_ = reinterpret_cast<tgk::FusedInstr*>(fake);
    input_region_ = fake + arena_bytes_ + 4096;
    for (int t : input_roots) ptr_[t] = input_region_ + input_offset_[t];
    workspace_ = reinterpret_cast<float*>(input_region_ + input_region_bytes_ + 4096);
    counters_ = reinterpret_cast<unsigned*>(fake + ((uintptr_t)1 << 39));
    partials_ = fake + ((uintptr_t)1 << 40);
    arena_ = nullptr;
    input_region_ = nullptr;
    return;
  }
  hip_check(hipMalloc(&input_region_, input_region_bytes_), "hipMalloc(inputs)");
  hip_check(hipHostMalloc(&staging_, input_region_bytes_, hipHostMallocDefault), "hipHostMalloc");
  memset(staging_, 0, input_region_bytes_);
  for (int t : input_roots) ptr_[t] = input_region_ + input_offset_[t];
  hip_check(hipHostMalloc(&loss_host_, 256, hipHostMallocDefault), "hipHostMalloc");
  if (workspace_bytes_) hip_check(hipMalloc(&workspace_, (workspace_bytes_ + 255) & ~(size_t)255), "hipMalloc(workspace)");
  if (partial_bytes_) hip_check(hipMalloc(&partials_, partial_bytes_), "hipMalloc(column partials)");
  if (counter_slots_) {
    hip_check(hipMalloc(&counters_, counter_slots_ * sizeof(unsigned)), "hipMalloc(counters)");
    hip_check(hipMemset(counters_, 0, counter_slots_ * sizeof(unsigned)), "hipMemset(counters)");
  }
  if (!fused_code_.empty()) {
    const size_t cb = fused_code_.size() * sizeof(tgk::FusedInstr);
    hip_check(hipMalloc(&fused_code_dev_, cb), "hipMalloc(fused code)");
    hip_check(hipMemcpy(fused_code_dev_, fused_code_.data(), cb, hipMemcpyHostToDevice), "hipMemcpy(fused code)");
  }
  // Zero everything once: params are uploaded by the caller, state starts at initValue.
  hip_check(hipMemset(arena_, 0, arena_bytes_), "hipMemset");
  for (auto& kv : state_tid_) {
    int t = kv.second;
    const tgj::Value& op = O(T_[t].src);
    double iv = op.at("initValue").num();
    if (iv != 0 && T_[t].dt == F32) tgk::fill(ptr_[t], tgk::DT_F32, iv, T_[t].numel, stream_);
    state_roots_.push_back(t);
  }
  hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
}

// Compile the generated group kernels (once per process; plan-only mode compiles them
// too, which proves they build, but loads nothing) and resolve each launch's function.
void Runtime::jit_finish() {
  if (jit_pending_.empty()) return;
  try {
    tgk::jit_compile(jit_pending_, !plan_only_);
    if (!plan_only_)
      for (auto& s : jit_slots_) s.fn = tgk::jit_function(s.name);
  } catch (const std::runtime_error& e) {
    throw Error(TG_INTERNAL, e.what());
  }
  jit_pending_.clear();
}

void Runtime::bind_all() {
  cur_counters_ = counters_;
  for (auto& n : init_nodes_) {
    for (int r : n.writes) if (!ptr_[r]) throw Error(TG_INTERNAL, "unallocated output in node " + n.kind);
    cur_ws_ = workspace_;
    n.launch = n.bind();
  }
  for (auto& n : nodes_) {
    for (int r : n.reads) if (!ptr_[r]) throw Error(TG_INTERNAL, "unallocated operand in node " + n.kind);
    for (int r : n.writes) if (!ptr_[r]) throw Error(TG_INTERNAL, "unallocated output in node " + n.kind);
    cur_ws_ = workspace_;
    n.launch = n.bind();
  }
  cur_ws_ = nullptr;
  cur_counters_ = nullptr;
}

// Bind the scratch-only launch list: nodes that use the workspace or the counters get
// new closures over the static scratch (workspace first, counters after it); the others
// share their regular closure. Runtimes whose workspace does not fit keep the reason.
void Runtime::prepare_noalloc() {
  const size_t ws = (workspace_bytes_ + 255) & ~(size_t)255;
  const size_t need = ws + (size_t)counter_slots_ * sizeof(unsigned);
  if (need > tg_kScratchBytes) {
    noalloc_error_ = "step_noalloc: this graph needs " + std::to_string(need) + " bytes of scratch; the limit is " +
                     std::to_string((size_t)tg_kScratchBytes);
    return;
  }
  char* base = scratch_address();
  noalloc_counters_ = reinterpret_cast<unsigned*>(base + ws);
  noalloc_launch_.clear();
  for (auto& n : nodes_) {
    if (!n.ws) { noalloc_launch_.push_back(n.launch); continue; }
    cur_ws_ = reinterpret_cast<float*>(base);
    cur_counters_ = noalloc_counters_;
    noalloc_launch_.push_back(n.bind());
  }
  cur_ws_ = nullptr;
  cur_counters_ = nullptr;
}

float Runtime::step_noalloc(int n, const char* const* names, const void* const* data, const int64_t* nbytes) {
  if (!opt_cfg_) throw Error(TG_INVALID_ARGUMENT, "step: graph has no optimizer (use run)");
  if (noalloc_launch_.size() != nodes_.size()) throw Error(TG_INVALID_ARGUMENT, noalloc_error_);
  std::lock_guard<std::mutex> g(g_noalloc_mu);
  advance_scalars(true);
  upload_inputs(n, names, data, nbytes, true);
  // The counters must start at zero; the scratch keeps whatever the last call left.
  if (counter_slots_) tgk::fill(noalloc_counters_, tgk::DT_I32, 0.0, counter_slots_, stream_);
  for (auto& f : noalloc_launch_) f(stream_);
  apply_copy_writebacks(stream_);
  hip_check(hipMemcpyAsync(loss_host_, dptr(outputs_.at(0)), 4, hipMemcpyDeviceToHost, stream_), "hipMemcpyAsync(D2H)");
  hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
  return loss_host_[0];
}

void Runtime::launch_all(hipStream_t st) {
  for (auto& n : nodes_) n.launch(st);
}

void Runtime::apply_copy_writebacks(hipStream_t st) {
  // Sources are computed from pre-step values, so all copies go after every kernel.
  for (auto& w : copy_writebacks_) {
    int dst = -1;
    auto ip = param_root.find(w.second);
    if (ip != param_root.end()) dst = ip->second;
    auto is = state_tid_.find(w.second);
    if (is != state_tid_.end()) dst = is->second;
    if (dst < 0) throw Error(TG_INVALID_ARGUMENT, "writeback destination '" + w.second + "' not found");
    int src = w.first;
    if (T_[src].numel != T_[dst].numel) throw Error(TG_INVALID_ARGUMENT, "writeback size mismatch for " + w.second);
    tgk::Strided sp{};
    const View& v = view_[src];
    Dims ds = contiguous_strides(v.dims);
    sp.rank = (int)v.dims.size();
    for (int d = 0; d < sp.rank; ++d) { sp.dims[d] = v.dims[d]; sp.s0[d] = ds[d]; sp.s1[d] = v.strides[d]; }
    if (sp.rank == 0) { sp.rank = 1; sp.dims[0] = 1; sp.s0[0] = 1; sp.s1[0] = 1; }
    tgk::strided_copy(ptr_[dst], ptr_[v.root], sp, T_[src].numel, st);
  }
}

// One execution of the step: a replay of the captured graph, or (graphs disabled) the
// same launches issued directly on the stream.
void Runtime::replay() {
  if (!use_graph_) {
    launch_all(stream_);
    apply_copy_writebacks(stream_);
    return;
  }
  ensure_graph();
  hip_check(hipGraphLaunch(graph_exec_, stream_), "hipGraphLaunch");
}

void Runtime::ensure_graph() {
  if (graph_exec_) return;
  hip_check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  try {
    launch_all(stream_);
    apply_copy_writebacks(stream_);
  } catch (...) {
    hipGraph_t g;
    hipStreamEndCapture(stream_, &g);
    if (g) hipGraphDestroy(g);
    throw;
  }
  hip_check(hipStreamEndCapture(stream_, &graph_), "hipStreamEndCapture");
  hip_check(hipGraphInstantiate(&graph_exec_, graph_, nullptr, nullptr, 0), "hipGraphInstantiate");
}

void Runtime::advance_scalars(bool optimizer) {
  // Per-step scalars (src/worker.ts:187-214), written into the host mirror of the tail of
  // the input region. The worker bumps t and the seed counter before the runtime checks
  // the inputs (src/worker.ts:225, :249), so a rejected call still consumes both.
  if (optimizer && opt_cfg_) {
    ++t_;
    double lr_now = resolve_lr(lr_, (double)t_);
    if (opt_kind_ == "adam") {
      double b1 = opt_cfg_->at("beta1").num(), b2 = opt_cfg_->at("beta2").num();
      float lrt = (float)(lr_now * std::sqrt(1 - std::pow(b2, (double)t_)) / (1 - std::pow(b1, (double)t_)));
      memcpy(staging_ + input_offset_[input_tid_.at(opt_cfg_->at("lrtInputName").str())], &lrt, 4);
      const tgj::Value& dn = opt_cfg_->at("decayShrinkInputName");
      if (!dn.null()) {
        float ds = (float)(1 - lr_now * opt_cfg_->at("weightDecay").num());
        memcpy(staging_ + input_offset_[input_tid_.at(dn.str())], &ds, 4);
      }
    } else {
      float lr = (float)lr_now;
      memcpy(staging_ + input_offset_[input_tid_.at(opt_cfg_->at("lrInputName").str())], &lr, 4);
    }
  }
  if (uses_prng_) {
    ++prng_counter_;
    int32_t s = (int32_t)(uint32_t)prng_counter_;
    memcpy(staging_ + input_offset_[input_tid_.at("__prngSeed")], &s, 4);
  }
}

void Runtime::upload_scalars() {
  if (input_region_bytes_ > user_bytes_)
    hip_check(hipMemcpyAsync(input_region_ + user_bytes_, staging_ + user_bytes_, input_region_bytes_ - user_bytes_,
                             hipMemcpyHostToDevice, stream_), "hipMemcpyAsync(H2D scalars)");
}

void Runtime::upload_inputs(int n, const char* const* names, const void* const* data, const int64_t* nbytes,
                            bool device) {
  // Validate the whole record before touching any state.
  std::map<int, int> given;   // input tid -> argument index
  for (int i = 0; i < n; ++i) {
    auto it = input_tid_.find(names[i]);
    if (it == input_tid_.end()) continue;   // extra inputs are ignored, as a JS record's would be
    int t = it->second;
    if (input_offset_[t] >= user_bytes_) continue;   // runtime-owned scalar: the worker overrides it
    if (nbytes[i] != T_[t].numel * 4)
      throw Error(TG_INVALID_ARGUMENT, std::string("input '") + names[i] + "': expected " +
                                           std::to_string(T_[t].numel * 4) + " bytes, got " + std::to_string(nbytes[i]));
    given[t] = i;
  }
  for (auto& kv : input_tid_)
    if (input_offset_[kv.second] < user_bytes_ && !given.count(kv.second))
      throw Error(TG_INVALID_ARGUMENT, "missing input '" + kv.first + "'");
  for (auto& g : given) {
    int t = g.first, i = g.second;
    if (device)
      hip_check(hipMemcpyAsync(input_region_ + input_offset_[t], data[i], (size_t)nbytes[i], hipMemcpyDeviceToDevice,
                               stream_), "hipMemcpyAsync(D2D)");
    else
      memcpy(staging_ + input_offset_[t], data[i], (size_t)nbytes[i]);
  }
  if (!device && user_bytes_)
    hip_check(hipMemcpyAsync(input_region_, staging_, user_bytes_, hipMemcpyHostToDevice, stream_), "hipMemcpyAsync(H2D)");
  upload_scalars();
}

// Device-resident batches for measurement and for callers that prefetch: slot k holds a
// copy of the user-input part of the input region.
void Runtime::stage_batch(int slot, int n, const char* const* names, const void* const* data, const int64_t* nbytes) {
  if (slot < 0 || slot > 4096) throw Error(TG_INVALID_ARGUMENT, "stage: slot out of range");
  if ((int)slots_.size() <= slot) slots_.resize(slot + 1, nullptr);
  if (!slots_[slot]) hip_check(hipMalloc(&slots_[slot], std::max<size_t>(user_bytes_, 256)), "hipMalloc(slot)");
  std::map<int, int> given;
  for (int i = 0; i < n; ++i) {
    auto it = input_tid_.find(names[i]);
    if (it == input_tid_.end() || input_offset_[it->second] >= user_bytes_) continue;
    if (nbytes[i] != T_[it->second].numel * 4) throw Error(TG_INVALID_ARGUMENT, std::string("stage: input '") + names[i] + "' has the wrong size");
    given[it->second] = i;
  }
  std::vector<char> host(std::max<size_t>(user_bytes_, 1), 0);
  for (auto& kv : input_tid_) {
    if (input_offset_[kv.second] >= user_bytes_) continue;
    auto g = given.find(kv.second);
    if (g == given.end()) throw Error(TG_INVALID_ARGUMENT, "stage: missing input '" + kv.first + "'");
    memcpy(host.data() + input_offset_[kv.second], data[g->second], (size_t)nbytes[g->second]);
  }
  if (user_bytes_) hip_check(hipMemcpy(slots_[slot], host.data(), user_bytes_, hipMemcpyHostToDevice), "hipMemcpy(slot)");
}

float Runtime::step_staged(int slot) {
  if (!opt_cfg_) throw Error(TG_INVALID_ARGUMENT, "step: graph has no optimizer (use run)");
  advance_scalars(true);
  if (slot < 0 || slot >= (int)slots_.size() || !slots_[slot]) throw Error(TG_INVALID_ARGUMENT, "step: slot not staged");
  if (user_bytes_)
    hip_check(hipMemcpyAsync(input_region_, slots_[slot], user_bytes_, hipMemcpyDeviceToDevice, stream_), "hipMemcpyAsync(D2D)");
  upload_scalars();
  replay();
  hip_check(hipMemcpyAsync(loss_host_, dptr(outputs_.at(0)), 4, hipMemcpyDeviceToHost, stream_), "hipMemcpyAsync(D2H)");
  hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
  return loss_host_[0];
}

float Runtime::step(int n, const char* const* names, const void* const* data, const int64_t* nbytes, bool device) {
  if (!opt_cfg_) throw Error(TG_INVALID_ARGUMENT, "step: graph has no optimizer (use run)");
  advance_scalars(true);
  upload_inputs(n, names, data, nbytes, device);
  replay();
  int lt = outputs_.at(0);
  hip_check(hipMemcpyAsync(loss_host_, dptr(lt), 4, hipMemcpyDeviceToHost, stream_), "hipMemcpyAsync(D2H)");
  hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
  return loss_host_[0];
}

void Runtime::run(int n, const char* const* names, const void* const* data, const int64_t* nbytes, void* out,
                  int64_t out_bytes) {
  // `run` injects only the PRNG seed (src/worker.ts:242-250); on a training graph the
  // optimizer's per-step scalar is then a missing input (src/runtime.ts:323-325).
  advance_scalars(false);
  if (opt_cfg_) {
    const char* f = opt_kind_ == "adam" ? "lrtInputName" : "lrInputName";
    throw Error(TG_INVALID_ARGUMENT, "tensorgrad: missing input '" + opt_cfg_->at(f).str() + "'");
  }
  upload_inputs(n, names, data, nbytes, false);
  replay();
  int o = outputs_.at(0);
  if (out_bytes != T_[o].numel * 4) throw Error(TG_INVALID_ARGUMENT, "run: output buffer has the wrong size");
  if (!view_[o].contiguous()) throw Error(TG_INTERNAL, "run: output is not contiguous");
  hip_check(hipMemcpyAsync(out, dptr(o), (size_t)out_bytes, hipMemcpyDeviceToHost, stream_), "hipMemcpyAsync(D2H)");
  hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
}

void Runtime::get_capture(const std::string& name, void* out, int64_t nbytes) {
  auto it = captures_.find(name);
  if (it == captures_.end()) throw Error(TG_INVALID_ARGUMENT, "capture '" + name + "' not registered");
  int t = it->second;
  if (nbytes != T_[t].numel * 4) throw Error(TG_INVALID_ARGUMENT, "capture '" + name + "': wrong byte size");
  hip_check(hipMemcpy(out, dptr(t), (size_t)nbytes, hipMemcpyDeviceToHost), "hipMemcpy(D2H)");
}

void Runtime::upload_params(int n, const char* const* names, const float* const* data, const int64_t* numel) {
  std::set<std::string> seen;
  for (int i = 0; i < n; ++i) {
    auto it = param_root.find(names[i]);
    if (it == param_root.end()) throw Error(TG_INVALID_ARGUMENT, std::string("uploadParams: unknown param '") + names[i] + "'");
    if (numel[i] != T_[it->second].numel)
      throw Error(TG_INVALID_ARGUMENT, std::string("uploadParams: '") + names[i] + "' expected " +
                                           std::to_string(T_[it->second].numel) + " floats, got " + std::to_string(numel[i]));
    seen.insert(names[i]);
  }
  for (auto& nm : param_names)
    if (!seen.count(nm)) throw Error(TG_INVALID_ARGUMENT, "uploadParams: missing param '" + nm + "'");
  for (int i = 0; i < n; ++i)
    hip_check(hipMemcpy(ptr_[param_root.at(names[i])], data[i], (size_t)numel[i] * 4, hipMemcpyHostToDevice), "hipMemcpy(H2D)");
}

void Runtime::download_params(int n, const char* const* names, float* const* data, const int64_t* numel) {
  hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
  for (int i = 0; i < n; ++i) {
    auto it = param_root.find(names[i]);
    if (it == param_root.end()) throw Error(TG_INVALID_ARGUMENT, std::string("downloadParams: unknown param '") + names[i] + "'");
    if (numel[i] != T_[it->second].numel) throw Error(TG_INVALID_ARGUMENT, "downloadParams: wrong size");
    hip_check(hipMemcpy(data[i], ptr_[it->second], (size_t)numel[i] * 4, hipMemcpyDeviceToHost), "hipMemcpy(D2H)");
  }
}

void Runtime::reset_optimizer() {
  for (int t : state_roots_) {
    double iv = O(T_[t].src).at("initValue").num();
    tgk::fill(ptr_[t], kdt(T_[t].dt), T_[t].dt == F32 ? iv : 0.0, T_[t].numel, stream_);
  }
  hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
  t_ = 0;
}

void Runtime::set_lr(const char* json) {
  if (!opt_cfg_) throw Error(TG_INVALID_ARGUMENT, "setLR: graph has no optimizer (compileForward graphs don't take optimizer state)");
  tgj::Value v;
  try { v = tgj::parse(json); } catch (std::exception& e) { throw Error(TG_INVALID_ARGUMENT, e.what()); }
  lr_ = rebase_lr(v, t_ + 1);
}

std::string Runtime::describe() {
  std::ostringstream o;
  o.precision(17);
  o << "{\"nodes\":[";
  for (size_t i = 0; i < nodes_.size(); ++i) {
    const Node& n = nodes_[i];
    o << (i ? "," : "") << "{\"kind\":\"" << n.kind << "\",\"op\":" << n.op << ",\"ir_kind\":\""
      << (n.op >= 0 ? kinds_[n.op] : "") << "\",\"shape\":\"" << n.shape << "\",\"flops\":" << n.flops
      << ",\"bytes\":" << n.bytes;
    if (!n.detail.empty()) o << ",\"ops\":\"" << n.detail << "\"";
    o << "}";
  }
  o << "],\"arena_bytes\":" << arena_bytes_ << ",\"workspace_bytes\":" << workspace_bytes_
    << ",\"ir_ops\":" << ops_.size() << "}";
  return o.str();
}

void Runtime::profile_nodes(int iters, double* ms, int64_t nout) {
  if (nout != (int64_t)nodes_.size()) throw Error(TG_INVALID_ARGUMENT, "profile: output length must equal node count");
  std::vector<hipEvent_t> ev(nodes_.size() + 1);
  for (auto& e : ev) hip_check(hipEventCreate(&e), "hipEventCreate");
  std::vector<double> acc(nodes_.size(), 0.0);
  for (int it = 0; it < iters; ++it) {
    hip_check(hipEventRecord(ev[0], stream_), "hipEventRecord");
    for (size_t i = 0; i < nodes_.size(); ++i) {
      nodes_[i].launch(stream_);
      hip_check(hipEventRecord(ev[i + 1], stream_), "hipEventRecord");
    }
    hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    for (size_t i = 0; i < nodes_.size(); ++i) {
      float m = 0;
      hip_check(hipEventElapsedTime(&m, ev[i], ev[i + 1]), "hipEventElapsedTime");
      acc[i] += m;
    }
  }
  for (auto& e : ev) hipEventDestroy(e);
  for (size_t i = 0; i < nodes_.size(); ++i) ms[i] = acc[i] / std::max(1, iters);
}

// Launch only the nodes whose kind is listed in `kinds` (comma separated; a leading '-'
// selects every node whose kind is NOT listed), in step order, `iters` times back to
// back between two HIP events on the runtime's stream. Returns milliseconds per pass and
// the number of nodes in a pass. The selected kernels read whatever the buffers hold.
// Per-node kernel time of eager steps: every kernel a node launches is dispatched with
// start / end events of its own (tgk::LaunchTimer), so the figure is the kernels' own
// durations, summed per node (split-K reductions with their GEMM), without the gaps
// between launches: the quantity a profiler's kernel trace reports.
void Runtime::profile_kernels(int iters, double* ms, int64_t nout) {
  if (nout != (int64_t)nodes_.size()) throw Error(TG_INVALID_ARGUMENT, "profile: output length must equal node count");
  tgk::LaunchTimer tm;
  tm.ev.resize(2 * (8 * nodes_.size() + 64));
  for (auto& e : tm.ev) hip_check(hipEventCreate(&e), "hipEventCreate");
  std::vector<double> acc(nodes_.size(), 0.0);
  std::vector<size_t> first(nodes_.size() + 1);
  try {
    for (int it = 0; it < iters; ++it) {
      tm.used = tm.missed = 0;
      tgk::launch_timer() = &tm;
      for (size_t i = 0; i < nodes_.size(); ++i) {
        first[i] = tm.used;
        nodes_[i].launch(stream_);
      }
      tgk::launch_timer() = nullptr;
      first[nodes_.size()] = tm.used;
      hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
      if (tm.missed) throw Error(TG_INTERNAL, "profile: kernel event pool exhausted");
      for (size_t i = 0; i < nodes_.size(); ++i)
        for (size_t k = first[i]; k < first[i + 1]; ++k) {
          float m = 0;
          hip_check(hipEventElapsedTime(&m, tm.ev[2 * k], tm.ev[2 * k + 1]), "hipEventElapsedTime");
          acc[i] += m;
        }
    }
  } catch (...) {
    tgk::launch_timer() = nullptr;
    hipStreamSynchronize(stream_);
    for (auto& e : tm.ev) hipEventDestroy(e);
    throw;
  }
  for (auto& e : tm.ev) hipEventDestroy(e);
  for (size_t i = 0; i < nodes_.size(); ++i) ms[i] = acc[i] / std::max(1, iters);
}

double Runtime::time_kinds(const std::string& kinds, int iters, int* launches) {
  bool negate = !kinds.empty() && kinds[0] == '-';
  std::set<std::string> want;
  std::stringstream ss(negate ? kinds.substr(1) : kinds);
  for (std::string k; std::getline(ss, k, ',');) if (!k.empty()) want.insert(k);
  std::vector<size_t> sel;
  for (size_t i = 0; i < nodes_.size(); ++i)
    if ((want.count(nodes_[i].kind) > 0) != negate) sel.push_back(i);
  *launches = (int)sel.size();
  if (sel.empty() || iters <= 0) return 0.0;
  hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
  hipEvent_t a, b;
  hip_check(hipEventCreate(&a), "hipEventCreate");
  hip_check(hipEventCreate(&b), "hipEventCreate");
  hip_check(hipEventRecord(a, stream_), "hipEventRecord");
  for (int it = 0; it < iters; ++it)
    for (size_t i : sel) nodes_[i].launch(stream_);
  hip_check(hipEventRecord(b, stream_), "hipEventRecord");
  hip_check(hipEventSynchronize(b), "hipEventSynchronize");
  float ms = 0;
  hip_check(hipEventElapsedTime(&ms, a, b), "hipEventElapsedTime");
  hipEventDestroy(a);
  hipEventDestroy(b);
  return ms / iters;
}

double Runtime::time_replays(int steps) {
  if (use_graph_) ensure_graph();
  hipEvent_t a, b;
  hip_check(hipEventCreate(&a), "hipEventCreate");
  hip_check(hipEventCreate(&b), "hipEventCreate");
  hip_check(hipEventRecord(a, stream_), "hipEventRecord");
  for (int i = 0; i < steps; ++i) replay();
  hip_check(hipEventRecord(b, stream_), "hipEventRecord");
  hip_check(hipEventSynchronize(b), "hipEventSynchronize");
  float ms = 0;
  hip_check(hipEventElapsedTime(&ms, a, b), "hipEventElapsedTime");
  hipEventDestroy(a);
  hipEventDestroy(b);
  return ms;
}

// Filled once by analyse() and never changed: readable without the runtime's lock.
const std::vector<std::string>& Runtime::state_names() const { return state_list_; }

int64_t Runtime::state_numel(const std::string& name) const {
  auto it = state_tid_.find(name);
  if (it == state_tid_.end()) throw Error(TG_INVALID_ARGUMENT, "optimizer state: unknown tensor '" + name + "'");
  return T_[it->second].numel;
}

void Runtime::download_state(int n, const char* const* names, float* const* data, const int64_t* numel) {
  hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
  for (int i = 0; i < n; ++i) {
    if (numel[i] != state_numel(names[i])) throw Error(TG_INVALID_ARGUMENT, std::string("optimizer state: '") + names[i] + "' has the wrong size");
    hip_check(hipMemcpy(data[i], ptr_[state_tid_.at(names[i])], (size_t)numel[i] * 4, hipMemcpyDeviceToHost), "hipMemcpy(D2H)");
  }
}

void Runtime::upload_state(int n, const char* const* names, const float* const* data, const int64_t* numel) {
  // Strict like uploadParams (src/runtime.ts:403-429): every state tensor exactly once.
  std::set<std::string> seen;
  for (int i = 0; i < n; ++i) {
    if (numel[i] != state_numel(names[i]))
      throw Error(TG_INVALID_ARGUMENT, std::string("optimizer state: '") + names[i] + "' expected " +
                                           std::to_string(state_numel(names[i])) + " elements, got " + std::to_string(numel[i]));
    if (!seen.insert(names[i]).second) throw Error(TG_INVALID_ARGUMENT, std::string("optimizer state: '") + names[i] + "' given twice");
  }
  for (auto& kv : state_tid_)
    if (!seen.count(kv.first)) throw Error(TG_INVALID_ARGUMENT, "optimizer state: missing tensor '" + kv.first + "'");
  hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
  for (int i = 0; i < n; ++i)
    hip_check(hipMemcpy(ptr_[state_tid_.at(names[i])], data[i], (size_t)numel[i] * 4, hipMemcpyHostToDevice), "hipMemcpy(H2D)");
}

// Checkpoint file: a safetensors container holding every parameter (F32, its shape),
// every optimizer state tensor (F32, or I32 for i32 state) and, in __metadata__, the
// optimizer kind, its step counter t and the PRNG seed counter, so that training
// resumed from it replays the same per-step scalars and dropout masks.
void Runtime::save_checkpoint(const std::string& path) {
  if (parent) throw Error(TG_INVALID_ARGUMENT, "checkpoint: a forward sibling shares its parent's params; save the parent");
  hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
  std::vector<tgst::OutTensor> ts;
  std::vector<int> tids;
  auto add = [&](const std::string& name, int t) {
    tgst::OutTensor o;
    o.name = name;
    o.dtype = T_[t].dt == F32 ? "F32" : "I32";
    o.shape = T_[t].shape;
    o.bytes = T_[t].numel * 4;
    ts.push_back(o);
    tids.push_back(t);
  };
  for (auto& nm : param_names) add(nm, param_root.at(nm));
  for (auto& kv : state_tid_) add(kv.first, kv.second);
  std::vector<std::pair<std::string, std::string>> meta = {
      {"format", "tensorgrad"}, {"tensorgrad.optimizer", opt_cfg_ ? opt_kind_ : std::string("none")},
      {"tensorgrad.step", std::to_string(t_)}, {"tensorgrad.prngCounter", std::to_string(prng_counter_)}};
  if (opt_cfg_) meta.emplace_back("tensorgrad.lr", tgj::dump(lr_));
  const std::string head = tgst::header(ts, meta);
  FILE* f = fopen(path.c_str(), "wb");
  if (!f) throw Error(TG_INVALID_ARGUMENT, "checkpoint: cannot open '" + path + "' for writing");
  bool ok = fwrite(head.data(), 1, head.size(), f) == head.size();
  std::vector<char> host;
  for (size_t i = 0; ok && i < ts.size(); ++i) {
    host.resize((size_t)ts[i].bytes);
    if (ts[i].bytes) {
      hipError_t e = hipMemcpy(host.data(), ptr_[tids[i]], (size_t)ts[i].bytes, hipMemcpyDeviceToHost);
      if (e != hipSuccess) { fclose(f); hip_check(e, "hipMemcpy(D2H checkpoint)"); }
    }
    ok = fwrite(host.data(), 1, host.size(), f) == host.size();
  }
  ok = (fclose(f) == 0) && ok;
  if (!ok) throw Error(TG_INVALID_ARGUMENT, "checkpoint: writing '" + path + "' failed");
}

// A checkpoint counter from __metadata__: decimal digits only, at most 18 of them.
static long long parse_counter(const std::string& v, const char* what) {
  if (v.empty() || v.size() > 18 || v.find_first_not_of("0123456789") != std::string::npos)
    throw Error(TG_INVALID_ARGUMENT, std::string("checkpoint: ") + what + " '" + v + "' is not a non-negative integer");
  return std::stoll(v);
}

static std::vector<uint8_t> read_file(const std::string& path) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) throw Error(TG_INVALID_ARGUMENT, "checkpoint: cannot open '" + path + "'");
  std::vector<uint8_t> buf;
  uint8_t chunk[1 << 16];
  size_t got;
  while ((got = fread(chunk, 1, sizeof chunk, f)) > 0) buf.insert(buf.end(), chunk, chunk + got);
  fclose(f);
  return buf;
}

// Everything a load would do, checked without touching the device: every parameter
// present with its shape; optimizer state all or nothing; no other tensors (integer and
// bool ones included); the counters and the LR schedule readable. Counters and the
// schedule are taken from the file only when it carries the optimizer state: a
// params-only file (e.g. converted pretrained weights) leaves all optimizer state alone.
Runtime::CkptPlan Runtime::check_checkpoint(const std::vector<uint8_t>& buf) const {
  if (parent) throw Error(TG_INVALID_ARGUMENT, "checkpoint: a forward sibling shares its parent's params; load into the parent");
  CkptPlan cp;
  try {
    cp.ix = tgst::parse(buf.data(), buf.size(), true);
  } catch (std::exception& e) {
    throw Error(TG_INVALID_ARGUMENT, e.what());
  }
  auto check = [&](const tgst::Entry& e, int t) {
    if (e.shape != T_[t].shape || e.dtype != (T_[t].dt == F32 ? "F32" : "I32"))
      throw Error(TG_INVALID_ARGUMENT, "checkpoint: tensor '" + e.name + "' does not match the graph's shape or dtype");
  };
  for (size_t i = 0; i < cp.ix.tensors.size(); ++i) {
    const tgst::Entry& e = cp.ix.tensors[i];
    auto p = param_root.find(e.name);
    auto s = state_tid_.find(e.name);
    if (p != param_root.end()) { check(e, p->second); cp.writes.emplace_back(i, p->second); }
    else if (s != state_tid_.end()) { check(e, s->second); cp.writes.emplace_back(i, s->second); ++cp.n_state; }
    else throw Error(TG_INVALID_ARGUMENT, "checkpoint: unknown tensor '" + e.name + "'");
  }
  for (const tgst::Entry& e : cp.ix.skipped)
    throw Error(TG_INVALID_ARGUMENT, "checkpoint: unknown tensor '" + e.name + "' (dtype " + e.dtype + ")");
  for (auto& nm : param_names)
    if (!cp.ix.find(nm)) throw Error(TG_INVALID_ARGUMENT, "checkpoint: missing param '" + nm + "'");
  if (cp.n_state && cp.n_state != state_tid_.size())
    throw Error(TG_INVALID_ARGUMENT, "checkpoint: holds part of the optimizer state (" + std::to_string(cp.n_state) +
                                         " of " + std::to_string(state_tid_.size()) + " tensors)");
  cp.t = t_;
  cp.c = prng_counter_;
  cp.lr = lr_;
  if (cp.n_state) {
    const std::string* k = cp.ix.meta("tensorgrad.optimizer");
    const std::string mine = opt_cfg_ ? opt_kind_ : std::string("none");
    if (k && *k != mine) throw Error(TG_INVALID_ARGUMENT, "checkpoint: optimizer '" + *k + "' does not match the graph's '" + mine + "'");
    const std::string* ts = cp.ix.meta("tensorgrad.step");
    if (!ts) throw Error(TG_INVALID_ARGUMENT, "checkpoint: optimizer state without a step counter");
    cp.t = parse_counter(*ts, "tensorgrad.step");
    if (const std::string* cs = cp.ix.meta("tensorgrad.prngCounter")) cp.c = parse_counter(*cs, "tensorgrad.prngCounter");
    if (const std::string* ls = cp.ix.meta("tensorgrad.lr"))
      if (opt_cfg_) {
        try {
          cp.lr = tgj::parse(ls->c_str());
        } catch (std::exception& e) {
          throw Error(TG_INVALID_ARGUMENT, std::string("checkpoint: lr: ") + e.what());
        }
      }
  }
  return cp;
}

std::string Runtime::check_checkpoint_file(const std::string& path) const {
  const std::vector<uint8_t> buf = read_file(path);
  const CkptPlan cp = check_checkpoint(buf);
  std::ostringstream o;
  o << "{\"params\":" << (cp.writes.size() - cp.n_state) << ",\"state\":" << cp.n_state
    << ",\"restoresCounters\":" << (cp.n_state ? "true" : "false") << ",\"step\":" << cp.t
    << ",\"prngCounter\":" << cp.c << "}";
  return o.str();
}

void Runtime::load_checkpoint(const std::string& path) {
  const std::vector<uint8_t> buf = read_file(path);
  const CkptPlan cp = check_checkpoint(buf);   // nothing is written unless the whole file checks out
  hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
  for (auto& w : cp.writes) {
    const tgst::Entry& e = cp.ix.tensors[w.first];
    if (e.end > e.begin)
      hip_check(hipMemcpy(ptr_[w.second], buf.data() + cp.ix.data_start + e.begin, (size_t)(e.end - e.begin),
                          hipMemcpyHostToDevice), "hipMemcpy(H2D checkpoint)");
  }
  t_ = cp.t;
  prng_counter_ = cp.c;
  lr_ = cp.lr;
}

}  // namespace tg

// ---- C ABI -------------------------------------------------------------------------------

struct tg_runtime {
  std::unique_ptr<tg::Runtime> rt;
  std::mutex mu;
  tg_runtime* parent = nullptr;
  std::vector<tg_runtime*> children;
};

namespace {
std::mutex g_registry_mu;
std::set<tg_runtime*> g_live;

template <class F>
tg_status guarded(F&& f) {
  try {
    f();
    tg::g_error.clear();
    return TG_OK;
  } catch (tg::Error& e) {
    tg::g_error = e.what();
    return e.code;
  } catch (std::exception& e) {
    tg::g_error = e.what();
    return TG_INTERNAL;
  }
}

bool live(tg_runtime* h) {
  std::lock_guard<std::mutex> g(g_registry_mu);
  return h && g_live.count(h);
}

// Names and sizes are fixed at creation. The getters take the registry lock, so a handle
// destroyed before or during the call answers 0 / NULL / -1 instead of being read; a
// returned name stays valid until the runtime is destroyed.
template <class R, class F>
R if_live(const tg_runtime* h, R dflt, F f) {
  std::lock_guard<std::mutex> g(g_registry_mu);
  if (!h || !g_live.count(const_cast<tg_runtime*>(h)) || !h->rt) return dflt;
  return f(*h->rt);
}
}  // namespace

extern "C" {

const char* tg_last_error(void) { return tg::g_error.c_str(); }

int tg_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

tg_status tg_runtime_create(const char* ir_json, tg_runtime** out) {
  if (!ir_json || !out) { tg::g_error = "null argument"; return TG_INVALID_ARGUMENT; }
  return guarded([&] {
    auto* h = new tg_runtime();
    try {
      h->rt.reset(new tg::Runtime(ir_json, nullptr));
    } catch (...) {
      delete h;
      throw;
    }
    std::lock_guard<std::mutex> g(g_registry_mu);
    g_live.insert(h);
    *out = h;
  });
}

tg_status tg_runtime_create_sibling(tg_runtime* parent, const char* ir_json, tg_runtime** out) {
  if (!live(parent)) { tg::g_error = "compileForward: parent graph not found"; return TG_INVALID_ARGUMENT; }
  return guarded([&] {
    auto* h = new tg_runtime();
    try {
      h->rt.reset(new tg::Runtime(ir_json, parent->rt.get()));
    } catch (...) {
      delete h;
      throw;
    }
    h->parent = parent;
    std::lock_guard<std::mutex> g(g_registry_mu);
    parent->children.push_back(h);
    g_live.insert(h);
    *out = h;
  });
}

static void destroy_rec(tg_runtime* h) {
  for (auto* c : h->children) destroy_rec(c);
  {
    std::lock_guard<std::mutex> lk(h->mu);
    h->rt.reset();
  }
  g_live.erase(h);
  delete h;
}

void tg_destroy(tg_runtime* h) {
  std::lock_guard<std::mutex> g(g_registry_mu);
  if (!h || !g_live.count(h)) return;
  if (h->parent && g_live.count(h->parent)) {
    auto& v = h->parent->children;
    v.erase(std::remove(v.begin(), v.end(), h), v.end());
  }
  destroy_rec(h);
}

#define TG_ENTER(h)                                                       \
  if (!live(h)) { tg::g_error = "graph destroyed"; return TG_ABORTED; } \
  std::lock_guard<std::mutex> lk_((h)->mu);                               \
  if (!(h)->rt) { tg::g_error = "graph destroyed"; return TG_ABORTED; }

int tg_param_count(const tg_runtime* h) {
  return if_live(h, 0, [](const tg::Runtime& r) { return (int)r.param_names.size(); });
}
const char* tg_param_name(const tg_runtime* h, int i) {
  return if_live(h, (const char*)nullptr, [i](const tg::Runtime& r) -> const char* {
    return i < 0 || i >= (int)r.param_names.size() ? nullptr : r.param_names[i].c_str();
  });
}
int64_t tg_param_numel(const tg_runtime* h, int i) {
  return if_live(h, (int64_t)-1, [i](const tg::Runtime& r) -> int64_t {
    return i < 0 || i >= (int)r.param_names.size() ? -1 : r.param_numel(i);
  });
}

tg_status tg_upload_params(tg_runtime* h, int n, const char* const* names, const float* const* data, const int64_t* numel) {
  TG_ENTER(h);
  return guarded([&] { h->rt->upload_params(n, names, data, numel); });
}

tg_status tg_download_params(tg_runtime* h, int n, const char* const* names, float* const* data, const int64_t* numel) {
  TG_ENTER(h);
  return guarded([&] { h->rt->download_params(n, names, data, numel); });
}

tg_status tg_step(tg_runtime* h, int n, const char* const* names, const void* const* data, const int64_t* nbytes,
                  float* loss) {
  TG_ENTER(h);
  return guarded([&] { float l = h->rt->step(n, names, data, nbytes, false); if (loss) *loss = l; });
}

tg_status tg_step_device(tg_runtime* h, int n, const char* const* names, const void* const* data, const int64_t* nbytes,
                         float* loss) {
  TG_ENTER(h);
  return guarded([&] { float l = h->rt->step(n, names, data, nbytes, true); if (loss) *loss = l; });
}

tg_status tg_step_noalloc(tg_runtime* h, int n, const char* const* names, const void* const* data,
                          const int64_t* nbytes, float* loss) {
  TG_ENTER(h);
  return guarded([&] { float l = h->rt->step_noalloc(n, names, data, nbytes); if (loss) *loss = l; });
}

tg_status tg_stage_batch(tg_runtime* h, int slot, int n, const char* const* names, const void* const* data,
                         const int64_t* nbytes) {
  TG_ENTER(h);
  return guarded([&] { h->rt->stage_batch(slot, n, names, data, nbytes); });
}

tg_status tg_step_staged(tg_runtime* h, int slot, float* loss) {
  TG_ENTER(h);
  return guarded([&] { float l = h->rt->step_staged(slot); if (loss) *loss = l; });
}

tg_status tg_run(tg_runtime* h, int n, const char* const* names, const void* const* data, const int64_t* nbytes,
                 void* out, int64_t out_bytes) {
  TG_ENTER(h);
  return guarded([&] { h->rt->run(n, names, data, nbytes, out, out_bytes); });
}

int tg_capture_count(const tg_runtime* h) {
  return if_live(h, 0, [](const tg::Runtime& r) { return (int)r.capture_names.size(); });
}
const char* tg_capture_name(const tg_runtime* h, int i) {
  return if_live(h, (const char*)nullptr, [i](const tg::Runtime& r) -> const char* {
    return i < 0 || i >= (int)r.capture_names.size() ? nullptr : r.capture_names[i].c_str();
  });
}

tg_status tg_get_capture(tg_runtime* h, const char* name, void* out, int64_t nbytes) {
  TG_ENTER(h);
  return guarded([&] { h->rt->get_capture(name, out, nbytes); });
}

tg_status tg_reset_optimizer(tg_runtime* h) {
  TG_ENTER(h);
  return guarded([&] { h->rt->reset_optimizer(); });
}

tg_status tg_set_lr(tg_runtime* h, const char* lr_json) {
  TG_ENTER(h);
  return guarded([&] { h->rt->set_lr(lr_json); });
}

int tg_state_count(tg_runtime* h) {
  return if_live(h, 0, [](const tg::Runtime& r) { return (int)r.state_names().size(); });
}
const char* tg_state_name(tg_runtime* h, int i) {
  return if_live(h, (const char*)nullptr, [i](const tg::Runtime& r) -> const char* {
    return i < 0 || i >= (int)r.state_names().size() ? nullptr : r.state_names()[i].c_str();
  });
}
int64_t tg_state_numel(tg_runtime* h, int i) {
  return if_live(h, (int64_t)-1, [i](const tg::Runtime& r) -> int64_t {
    return i < 0 || i >= (int)r.state_names().size() ? -1 : r.state_numel(r.state_names()[i]);
  });
}

tg_status tg_download_state(tg_runtime* h, int n, const char* const* names, float* const* data, const int64_t* numel,
                            int64_t* step_t, int64_t* prng_counter) {
  TG_ENTER(h);
  return guarded([&] {
    h->rt->download_state(n, names, data, numel);
    if (step_t) *step_t = h->rt->step_count();
    if (prng_counter) *prng_counter = h->rt->prng_count();
  });
}

tg_status tg_upload_state(tg_runtime* h, int n, const char* const* names, const float* const* data, const int64_t* numel,
                          int64_t step_t, int64_t prng_counter) {
  TG_ENTER(h);
  return guarded([&] {
    if (step_t < 0 || prng_counter < 0) throw tg::Error(TG_INVALID_ARGUMENT, "optimizer state: counters must be >= 0");
    h->rt->upload_state(n, names, data, numel);
    h->rt->set_counters(step_t, prng_counter);
  });
}

tg_status tg_save_checkpoint(tg_runtime* h, const char* path) {
  if (!path) { tg::g_error = "null argument"; return TG_INVALID_ARGUMENT; }
  TG_ENTER(h);
  return guarded([&] { h->rt->save_checkpoint(path); });
}

tg_status tg_load_checkpoint(tg_runtime* h, const char* path) {
  if (!path) { tg::g_error = "null argument"; return TG_INVALID_ARGUMENT; }
  TG_ENTER(h);
  return guarded([&] { h->rt->load_checkpoint(path); });
}

tg_status tg_check_checkpoint(const char* ir_json, const char* path, char* out, int64_t out_len) {
  if (!ir_json || !path || !out || out_len <= 0) { tg::g_error = "null argument"; return TG_INVALID_ARGUMENT; }
  return guarded([&] {
    tg::Runtime r(ir_json, nullptr, true);
    const std::string s = r.check_checkpoint_file(path);
    if ((int64_t)s.size() + 1 > out_len) throw tg::Error(TG_INVALID_ARGUMENT, "check_checkpoint: output buffer too small");
    memcpy(out, s.c_str(), s.size() + 1);
  });
}

tg_status tg_safetensors_index(const void* buf, int64_t len, char* out, int64_t out_len) {
  if (!buf || !out || len < 0) { tg::g_error = "null argument"; return TG_INVALID_ARGUMENT; }
  return guarded([&] {
    tgst::Index ix;
    try {
      ix = tgst::parse(static_cast<const uint8_t*>(buf), (uint64_t)len);
    } catch (std::exception& e) {
      throw tg::Error(TG_INVALID_ARGUMENT, e.what());
    }
    std::string o = "{\"dataStart\":" + std::to_string(ix.data_start) + ",\"tensors\":[";
    auto entry = [&](const tgst::Entry& e) {
      std::string s = "{\"name\":" + tgst::quote(e.name) + ",\"dtype\":" + tgst::quote(e.dtype) + ",\"shape\":[";
      for (size_t i = 0; i < e.shape.size(); ++i) s += (i ? "," : "") + std::to_string(e.shape[i]);
      return s + "],\"begin\":" + std::to_string(e.begin) + ",\"end\":" + std::to_string(e.end) + "}";
    };
    for (size_t i = 0; i < ix.tensors.size(); ++i) o += (i ? "," : "") + entry(ix.tensors[i]);
    o += "],\"skipped\":[";
    for (size_t i = 0; i < ix.skipped.size(); ++i) o += (i ? "," : "") + entry(ix.skipped[i]);
    o += "],\"metadata\":{";
    for (size_t i = 0; i < ix.metadata.size(); ++i)
      o += (i ? "," : "") + tgst::quote(ix.metadata[i].first) + ":" + tgst::quote(ix.metadata[i].second);
    o += "}}";
    if ((int64_t)o.size() + 1 > out_len) throw tg::Error(TG_INVALID_ARGUMENT, "safetensors index: output buffer too small");
    memcpy(out, o.c_str(), o.size() + 1);
  });
}

tg_status tg_plan(const char* ir_json, char* buf, int64_t buflen) {
  if (!ir_json || !buf) { tg::g_error = "null argument"; return TG_INVALID_ARGUMENT; }
  return guarded([&] {
    tg::Runtime rt(ir_json, nullptr, true);
    std::string s = rt.describe();
    if ((int64_t)s.size() + 1 > buflen) throw tg::Error(TG_INVALID_ARGUMENT, "plan: buffer too small (" + std::to_string(s.size() + 1) + ")");
    memcpy(buf, s.c_str(), s.size() + 1);
  });
}

tg_status tg_describe(tg_runtime* h, char* buf, int64_t buflen) {
  TG_ENTER(h);
  return guarded([&] {
    std::string s = h->rt->describe();
    if ((int64_t)s.size() + 1 > buflen) throw tg::Error(TG_INVALID_ARGUMENT, "describe: buffer too small (" + std::to_string(s.size() + 1) + ")");
    memcpy(buf, s.c_str(), s.size() + 1);
  });
}

tg_status tg_profile_nodes(tg_runtime* h, int iters, double* ms_out, int64_t n_out) {
  TG_ENTER(h);
  return guarded([&] { h->rt->profile_nodes(iters, ms_out, n_out); });
}

tg_status tg_profile_kernels(tg_runtime* h, int iters, double* ms_out, int64_t n_out) {
  TG_ENTER(h);
  return guarded([&] { h->rt->profile_kernels(iters, ms_out, n_out); });
}

tg_status tg_time_replays(tg_runtime* h, int steps, double* total_ms) {
  TG_ENTER(h);
  return guarded([&] { *total_ms = h->rt->time_replays(steps); });
}

tg_status tg_time_kinds(tg_runtime* h, const char* kinds, int iters, double* ms_per_pass, int* launches) {
  TG_ENTER(h);
  return guarded([&] { *ms_per_pass = h->rt->time_kinds(kinds ? kinds : "", iters, launches); });
}

}  // extern "C"
