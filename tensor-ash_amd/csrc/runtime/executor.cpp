// Executor: validation -> routing -> HIP launches on a slot's stream.
//
// Replaces src/executor/{mod,dispatch,validation,recording,splitk2,
// reduction,tuning,prepared,submission,slot,transfer}.rs.  Vulkan command
// buffers, fences and timestamp queries become a HIP stream per slot,
// hipEvents and, for prepared replay, an instantiated hipGraph.  Stream
// order already serialises the ops of one submission, which is exactly
// the hazard rule of run_op_graph (recording/graph.rs:40-137): a later op
// sees every earlier op's writes.
#include <algorithm>
#include <atomic>
#include <cctype>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <deque>
#include <cstring>
#include <fstream>
#include <functional>
#include <sstream>
#include <sys/stat.h>
#include <unistd.h>

#include "internal.hpp"

namespace tensor_ash {

namespace {

uint32_t div_ceil(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// Device scratch owned by a slot or by a prepared graph.  Ops of one
// submission run in stream order, so they can share one region.
struct Scratch {
  void *splitk = nullptr;
  uint64_t splitk_bytes = 0;
  void *partial = nullptr;
  uint64_t partial_bytes = 0;
  uint32_t *counters = nullptr;
  uint64_t counters_len = 0;
  // Decode-MLP region (generation words + tagged hand-off words), used by
  // no other kernel and zeroed when allocated or reset.
  void *mlp = nullptr;
  uint64_t mlp_bytes = 0;
  // f16 copy of a dual SwiGLU launch's output for the next op's A (kept
  // apart from the split-K region, which holds the dual launch's own A).
  void *shadow = nullptr;
  uint64_t shadow_bytes = 0;
  // Grid-barrier words of the persistent GEMV chain (arrival count,
  // generation; zeroed once, the count returns to zero after every
  // barrier).  Kept apart from `counters`, whose tile counters must all
  // read zero between launches.
  uint32_t *barrier = nullptr;

  void release() {
    if (splitk)
      (void)hipFree(splitk);
    if (partial)
      (void)hipFree(partial);
    if (counters)
      (void)hipFree(counters);
    if (mlp)
      (void)hipFree(mlp);
    if (shadow)
      (void)hipFree(shadow);
    if (barrier)
      (void)hipFree(barrier);
    splitk = partial = mlp = shadow = nullptr;
    counters = barrier = nullptr;
    splitk_bytes = partial_bytes = counters_len = mlp_bytes = shadow_bytes = 0;
  }
  void ensure_barrier(bool want) {
    if (!want || barrier)
      return;
    hip_check(device_malloc(reinterpret_cast<void **>(&barrier), 2 * TA_GEMV_COUNTER_STRIDE * 4),
              "hipMalloc (GEMV chain barrier)");
    hip_check(hipMemset(barrier, 0, 2 * TA_GEMV_COUNTER_STRIDE * 4), "hipMemset (GEMV chain barrier)");
  }
  void ensure_shadow(uint64_t bytes) {
    if (bytes <= shadow_bytes)
      return;
    if (shadow)
      hip_check(hipFree(shadow), "hipFree");
    shadow = nullptr;
    hip_check(device_malloc(&shadow, bytes), "hipMalloc (f16 output copy)");
    shadow_bytes = bytes;
  }
  void ensure_mlp(uint64_t bytes) {
    if (bytes <= mlp_bytes)
      return;
    if (mlp)
      hip_check(hipFree(mlp), "hipFree");
    mlp = nullptr;
    hip_check(device_malloc(&mlp, bytes), "hipMalloc (decode-MLP scratch)");
    mlp_bytes = bytes;
    reset_mlp();
  }
  // Zeroed again after a launch that gave up waiting (its hand-off words
  // may carry the generation the next launch would use).
  void reset_mlp() {
    if (mlp)
      hip_check(hipMemset(mlp, 0, mlp_bytes), "hipMemset (decode-MLP scratch)");
  }
  // Grow to at least the given sizes.  Counters start at zero (the GEMV
  // kernels reset them themselves after use).
  void ensure(uint64_t sk_bytes, uint64_t part_bytes, uint64_t n_counters) {
    if (sk_bytes > splitk_bytes) {
      if (splitk)
        hip_check(hipFree(splitk), "hipFree");
      splitk = nullptr;
      hip_check(device_malloc(&splitk, sk_bytes), "hipMalloc (split-K scratch)");
      splitk_bytes = sk_bytes;
    }
    if (part_bytes > partial_bytes) {
      if (partial)
        hip_check(hipFree(partial), "hipFree");
      partial = nullptr;
      hip_check(device_malloc(&partial, part_bytes), "hipMalloc (GEMV partials)");
      partial_bytes = part_bytes;
    }
    if (n_counters > counters_len) {
      if (counters)
        hip_check(hipFree(counters), "hipFree");
      counters = nullptr;
      hip_check(device_malloc(reinterpret_cast<void **>(&counters), n_counters * 4),
                "hipMalloc (GEMV counters)");
      hip_check(hipMemset(counters, 0, n_counters * 4), "hipMemset (GEMV counters)");
      counters_len = n_counters;
    }
  }
};

// Extra stream of a slot for run_ops' independent ops: its own scratch,
// so ops on different lanes never share partial planes or counters.
struct SideLane {
  hipStream_t stream = nullptr;
  hipEvent_t done = nullptr;
  Scratch scratch;
};

// Streams a submission of independent ops is spread over (the slot's own
// plus three side lanes): GPU_MAX_HW_QUEUES is 4 per process by default.
constexpr size_t kRunOpsLanes = 4;

struct Slot {
  hipStream_t stream = nullptr;
  hipEvent_t start = nullptr, end = nullptr;
  Scratch scratch;
  uint32_t *host_status = nullptr; // mapped pinned word (decode-MLP status)
  hipEvent_t fork = nullptr;       // created with the side lanes
  std::vector<SideLane> side;      // created on first use
};

// Mapped pinned word the decode-MLP kernel reports its wait status into.
uint32_t *alloc_host_status() {
  void *p = nullptr;
  hip_check(host_malloc(&p, 64, hipHostMallocMapped), "hipHostMalloc");
  *static_cast<volatile uint32_t *>(p) = 0;
  return static_cast<uint32_t *>(p);
}

// Device address of a status word, looked up once per word: the runtime
// call sits between a submission's start event and its first launch.
uint32_t *device_status(uint32_t *host) {
  static std::mutex mu;
  static std::map<uint32_t *, uint32_t *> cache;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(host);
  if (it != cache.end())
    return it->second;
  void *dp = nullptr;
  hip_check(hipHostGetDevicePointer(&dp, host, 0), "hipHostGetDevicePointer");
  cache[host] = static_cast<uint32_t *>(dp);
  return static_cast<uint32_t *>(dp);
}

void check_host_status(uint32_t *word, void *mlp, uint64_t mlp_bytes) {
  volatile uint32_t *w = word;
  if (*w != 0) {
    *w = 0;
    if (mlp)
      hip_check(hipMemset(mlp, 0, mlp_bytes), "hipMemset (decode-MLP scratch)");
    fail("persistent launch (decode MLP or GEMV chain): a workgroup gave up waiting for its "
         "inputs");
  }
}

// Complete route for one op (src/executor/mod.rs:125-139).
struct OpPlan {
  size_t kernel = 0;
  std::optional<uint32_t> splitk2;
  // Launch role: 0 = normal, 1 = fused into the next op's dual GEMV,
  // 2 = dual GEMV that also produces the previous op's output,
  // 3 = decode-MLP launch covering this op and the next 3 * mlp_layers - 1,
  // 4 = covered, 5 = persistent GEMV-chain launch covering this op and the
  // next chain_jobs - 1, 6 = covered by it.
  int role = 0;
  uint32_t mlp_layers = 0;
  uint32_t chain_jobs = 0;
};

struct ScratchNeed {
  uint64_t splitk = 0, partial = 0, counters = 0, mlp = 0, shadow = 0;
  bool barrier = false;
  void merge(const ScratchNeed &o) {
    barrier = barrier || o.barrier;
    shadow = std::max(shadow, o.shadow);
    splitk = std::max(splitk, o.splitk);
    partial = std::max(partial, o.partial);
    counters = std::max(counters, o.counters);
    mlp = std::max(mlp, o.mlp);
  }
};

// One model-op launch, planned (validated, arguments packed) before
// anything is recorded.
struct ElemLaunch {
  std::string symbol;
  uint32_t groups = 0, gy = 1, threads = 256;
  std::vector<uint8_t> args;
};
// A model op: one launch, or several in stream order (decode attention).
using ElemLaunches = std::vector<ElemLaunch>;

} // namespace

struct ExecutorImpl;
ElemLaunches plan_exec_elem(ExecutorImpl &e, const ExecOp &op);
void check_gemv_chain(const ExecutorImpl &e, const std::vector<MatmulOp> &jobs);

struct ExecutorImpl {
  std::shared_ptr<Context> ctx;
  KernelSelection selection;
  ExecutorConfig config;
  std::mutex slots_mu;
  std::condition_variable slot_cv;
  std::deque<Slot *> free_slots;
  std::vector<Slot *> all_slots;

  mutable std::mutex tuned_mu;
  std::map<TuneKey, TuneEntry> tuned;
  std::string header;

  // ---- slots (src/executor/submission.rs:37-55) ----
  Slot *checkout() {
    std::unique_lock<std::mutex> lock(slots_mu);
    slot_cv.wait(lock, [&] { return !free_slots.empty(); });
    Slot *s = free_slots.front();
    free_slots.pop_front();
    return s;
  }
  void give_back(Slot *s) {
    {
      std::lock_guard<std::mutex> lock(slots_mu);
      free_slots.push_back(s);
    }
    slot_cv.notify_one();
  }
  struct Lease {
    ExecutorImpl *e;
    Slot *s;
    explicit Lease(ExecutorImpl *ex) : e(ex), s(ex->checkout()) {}
    ~Lease() { e->give_back(s); }
  };

  // ---- validation (src/executor/validation.rs) ----
  void validate_tensor(const Tensor *t, const char *role) const {
    if (!t)
      fail(std::string(role) + " tensor is null");
    if (!t->belongs_to(ctx.get()))
      fail(std::string(role) + " tensor belongs to a different HIP context");
  }
  void validate_call(const MatmulCall &c) const {
    validate_tensor(c.a, "A");
    validate_tensor(c.b, "B");
    validate_tensor(c.c, "C");
    if (c.c->buffer_id() == c.a->buffer_id() || c.c->buffer_id() == c.b->buffer_id())
      fail("C must not alias A or B; in-place matmul is not supported");
  }
  void validate_op(const MatmulOp &op) const {
    validate_call(op.call);
    if (op.epilogue.bias)
      validate_tensor(op.epilogue.bias, "bias");
    if (op.epilogue.binary.kind != EpilogueBinary::Kind::None)
      validate_tensor(op.epilogue.binary.d, "D");
    if (op.normed_a)
      validate_tensor(op.normed_a->weight, "normed-A weight");
    if (op.store.table)
      validate_tensor(op.store.table, "store rope table");
    if (op.store.dst)
      validate_tensor(op.store.dst, "store destination");
  }

  // ---- routing (src/pipeline/mod.rs:259-288, executor/mod.rs:179-315) ----
  std::optional<TuneEntry> tuned_entry(const TuneKey &key) const {
    std::lock_guard<std::mutex> lock(tuned_mu);
    auto it = tuned.find(key);
    if (it == tuned.end())
      return std::nullopt;
    return it->second;
  }

  OpPlan plan_shape(uint32_t batch, uint32_t m, uint32_t n, uint32_t k, bool b_f16,
                    bool splitk_eligible) const {
    OpPlan plan;
    std::optional<std::optional<uint32_t>> tuned_splits;
    if (selection.index) {
      plan.kernel = *selection.index;
    } else if (auto e = tuned_entry(TuneKey{batch, m, n, k, b_f16})) {
      plan.kernel = e->kernel;
      tuned_splits = e->splitk2_splits;
    } else {
      plan.kernel = heuristic_kernel_index(ctx->cu_count(), batch, m, n, k, b_f16, false);
    }
    if (splitk_eligible && !b_f16 && selection.is_auto()) {
      std::optional<uint32_t> splits =
          tuned_splits ? *tuned_splits : heuristic_splits(ctx->cu_count(), batch, m, n, k);
      if (splits && auto_route_fits(batch, m, n, k, *splits)) {
        plan.splitk2 = splits;
        // Stage 1 runs on the split-K tile of run_matmuls_split_k2 (and of
        // dispatch_info_for), so an op gives the same bits whether it is
        // submitted alone or together with others.
        plan.kernel = registry_index(splitk_stage1_spec(m, n, k).name);
      }
    }
    return plan;
  }

  // Auto routes whose kernel cannot honour an op's decode fusions fall
  // back onto the heuristic pick when that one can (src/executor/mod.rs:
  // 259-315, demote_for_op); explicit selections keep their loud failure
  // at record time.
  OpPlan plan_op(const MatmulOp &op, const ResolvedMatmul &d, bool splitk_eligible) const {
    OpPlan plan = plan_matmul(d, splitk_eligible && !op.has_decode_fusion());
    if (op.has_decode_fusion() && selection.is_auto() && !fusions_fit(op, plan.kernel)) {
      const size_t h = heuristic_kernel_index(ctx->cu_count(), d.batch, d.m, d.n, d.k, d.b_f16,
                                              d.packed_b, d.a_f16);
      if (fusions_fit(op, h)) {
        plan.kernel = h;
        plan.splitk2.reset();
      }
    }
    return plan;
  }
  static bool fusions_fit(const MatmulOp &op, size_t kernel) {
    const KernelSpec &s = KERNEL_SPECS[kernel];
    return (!op.normed_a || s.supports_normed_a()) && (op.store.is_none() || s.supports_store());
  }

  OpPlan plan_matmul(const ResolvedMatmul &d, bool splitk_eligible) const {
    if (d.packed_b) {
      OpPlan p;
      p.kernel = heuristic_kernel_index(ctx->cu_count(), d.batch, d.m, d.n, d.k, true, true);
      return p;
    }
    if (d.a_f16) {
      // The a16 kernels are the only f16-activation route: a fixed pick,
      // outside tuning and split-K (src/executor/mod.rs:218-257).
      OpPlan p;
      p.kernel = heuristic_kernel_index(ctx->cu_count(), d.batch, d.m, d.n, d.k, true, false, true);
      if (selection.index && kernel_supports(KERNEL_SPECS[*selection.index], d))
        p.kernel = *selection.index;
      return p;
    }
    return plan_shape(d.batch, d.m, d.n, d.k, d.b_f16, splitk_eligible);
  }

  // ---- launches ----
  void launch(const std::string &symbol, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t threads,
              void *args, hipStream_t stream, void *args2 = nullptr) const {
    hipFunction_t f = static_cast<hipFunction_t>(ctx->function(symbol));
    void *params[] = {args, args2};
    hip_check(hipModuleLaunchKernel(f, gx, gy, gz, threads, 1, 1, 0, stream, params, nullptr),
              ("launch " + symbol).c_str());
  }

  ScratchNeed scratch_need(const ResolvedMatmul &d, const OpPlan &p) const {
    ScratchNeed need;
    const KernelSpec &s = KERNEL_SPECS[p.kernel];
    if (p.splitk2) {
      need.splitk = (uint64_t)d.batch * d.m * d.n * *p.splitk2 *
                    splitk_sub_splits(ctx->cu_count(), d, *p.splitk2) * 4;
    } else if (s.is_gemv()) {
      GemvPlan g = plan_gemv(ctx->cu_count(), d.m, d.n, d.k, s.tile_n, p.role == 2,
                            gemv_unit(s.tile_n, s.kind == KernelKind::GemvF32Row, p.role == 2, d.m));
      need.partial = g.partial_bytes;
      need.counters = (uint64_t)g.tiles * TA_GEMV_COUNTER_STRIDE;
    } else if (s.kind == KernelKind::GemmF16Mfma && gemm_lds_ok(d)) {
      need.splitk = 2 * a16_bytes(d); // two f16 copies of A (CvtCache)
    } else if (s.kind == KernelKind::GemmF16Sk) {
      need.splitk = 2 * a16_bytes(d);
      const uint32_t splits = h16sk_splits(ctx->cu_count(), d.batch, d.m, d.n, d.k, s.tile_m, s.tile_n);
      if (splits > 1) {
        const uint64_t tiles =
            (uint64_t)d.batch * div_ceil(d.m, s.tile_m) * div_ceil(d.n, s.tile_n);
        need.partial = tiles * splits * s.tile_m * s.tile_n * 4;
        need.counters = tiles * TA_GEMV_COUNTER_STRIDE;
      }
    }
    return need;
  }

  // f16 copy of A for the pipelined f16w route (one plane when A is
  // broadcast), kept in the split-K region: ops run in stream order.
  static uint64_t a16_bytes(const ResolvedMatmul &d) {
    const uint64_t planes = d.batch_stride_a ? d.batch : 1;
    return (planes * d.m * d.k * 2 + 255) / 256 * 256;
  }

  // f16 copies of A that pre-passes (or a dual launch's f16 output copy)
  // of a submission left behind: a later f16w GEMM with the same A (same
  // buffer, same elements) reuses one unless an op in between wrote that
  // buffer, or wrote the split-K region the copy lives in (record() and
  // launch_gemm() drop such entries).  Two entries, so a layer that
  // converts x for QKV and then the attention output for O still finds x
  // for its up/gate pair.  Pre-pass copies go to the half of the split-K
  // region the other live copy does not use (scratch_need reserves two
  // halves, each as large as the op's A).
  struct CvtEntry {
    const void *buffer = nullptr;
    const void *src = nullptr;
    uint64_t n = 0;
    void *base = nullptr;       // where the copy lives
    size_t producer = SIZE_MAX; // op whose epilogue wrote it, if any
    int half = -1;              // split-K region half, -1 = elsewhere
    uint64_t age = 0;
  };
  struct CvtCache {
    CvtEntry e[2];
    uint64_t clock = 0;
    CvtEntry *find(const void *buffer, const void *src, uint64_t n) {
      for (auto &x : e)
        if (x.buffer && x.buffer == buffer && x.src == src && x.n == n)
          return &x;
      return nullptr;
    }
    // The entry to replace: an empty one, else the older.
    CvtEntry &victim() {
      if (!e[0].buffer)
        return e[0];
      if (!e[1].buffer)
        return e[1];
      return e[0].age <= e[1].age ? e[0] : e[1];
    }
    // A copy written at `v.base` replaces whatever entry that memory held
    // (every dual launch writes its f16 output copy to the same scratch).
    void put(CvtEntry &slot, CvtEntry v) {
      for (auto &x : e)
        if (&x != &slot && x.buffer && x.base == v.base)
          x = CvtEntry{};
      v.age = ++clock;
      slot = v;
    }
    // An op wrote `buffer`: copies of it are stale (except the one that
    // op's own epilogue produced).
    void wrote(const void *buffer, size_t op) {
      for (auto &x : e)
        if (x.buffer && x.buffer == buffer && x.producer != op)
          x = CvtEntry{};
    }
    void drop_region() { // the split-K region was overwritten
      for (auto &x : e)
        if (x.half >= 0)
          x = CvtEntry{};
    }
  };

  // Does op i take the f32 -> f16 pre-pass of its A (the pipelined f16w
  // route; not a16, whose A is f16 already)?
  bool converts_a(const ResolvedMatmul &d, const OpPlan &p) const {
    if (p.role == 1 || p.role == 3 || p.role == 4 || p.role == 5 || p.role == 6 || p.splitk2)
      return false;
    const KernelSpec &s = KERNEL_SPECS[p.kernel];
    return (s.kind == KernelKind::GemmF16Mfma || s.kind == KernelKind::GemmF16Sk) &&
           gemm_lds_ok(d);
  }

  // The first two distinct A's of a submission that take the pre-pass and
  // that no earlier op writes (inputs, so converting them first changes no
  // value) are converted by one launch into the two halves of the copy
  // region and entered in the cache, where the ops then find them: one
  // launch instead of two on the submission's critical path (the prefill
  // layer converts x for QKV and up/gate and the attention output for O).
  // Not with split-K ops in the submission: their planes share the region.
  void convert_inputs_up_front(const std::vector<MatmulOp> &ops,
                               const std::vector<ResolvedMatmul> &res,
                               const std::vector<OpPlan> &plans, Scratch &scratch, CvtCache &cvt,
                               hipStream_t stream) const {
    if (std::getenv("TA_NO_CVT_PAIR"))
      return;
    for (const auto &p : plans)
      if (p.splitk2)
        return;
    std::vector<CvtCandidate> cand(ops.size());
    for (size_t i = 0; i < ops.size(); ++i) {
      const MatmulOp &op = ops[i];
      cand[i].a_buffer = op.call.a->buffer_id();
      cand[i].a_ptr = op.call.a->device_ptr();
      cand[i].n = (res[i].batch_stride_a ? (uint64_t)res[i].batch : 1) * res[i].m * res[i].k;
      cand[i].converts = converts_a(res[i], plans[i]);
      cand[i].writes[0] = op.call.c->buffer_id();
      cand[i].writes[1] = op.store.dst ? op.store.dst->buffer_id() : nullptr;
    }
    const std::vector<size_t> picks = paired_conversion_picks(cand);
    if (picks.size() != 2)
      return;
    CvtArgs job[2];
    const void *bufs[2];
    for (int j = 0; j < 2; ++j) {
      const CvtCandidate &c = cand[picks[j]];
      job[j] = CvtArgs{static_cast<const float *>(c.a_ptr), nullptr, c.n};
      bufs[j] = c.a_buffer;
    }
    const uint64_t half_bytes = scratch.splitk_bytes / 2 / 256 * 256;
    for (int j = 0; j < 2; ++j)
      if ((job[j].n * 2 + 255) / 256 * 256 > half_bytes)
        return;
    CvtPairArgs pa{};
    for (int j = 0; j < 2; ++j) {
      pa.job[j] = job[j];
      pa.job[j].dst = reinterpret_cast<uint16_t *>(static_cast<char *>(scratch.splitk) +
                                                   j * half_bytes);
    }
    pa.blocks0 = (job[0].n + 8 * 256 - 1) / (8 * 256);
    const uint64_t blocks = pa.blocks0 + (job[1].n + 8 * 256 - 1) / (8 * 256);
    if (blocks > 0x7fffffffull)
      return;
    launch("ta_cvt_f32_f16_pair", (uint32_t)blocks, 1, 1, 256, &pa, stream);
    for (int j = 0; j < 2; ++j)
      cvt.put(cvt.e[j], CvtEntry{bufs[j], pa.job[j].src, job[j].n, pa.job[j].dst, SIZE_MAX, j});
  }

  // Does op i (the gate of a dual SwiGLU launch) feed op i + 1 as A on the
  // f16w pipelined route?  Then the dual launch also writes an f16 copy of
  // its output (the conversion pre-pass's values: the same RNE rounding of
  // the same f32 results) and op i + 1 reads that instead of converting.
  static bool f16_copy_feeds_next(const std::vector<MatmulOp> &ops,
                                  const std::vector<ResolvedMatmul> &res,
                                  const std::vector<OpPlan> &plans, size_t i) {
    const size_t j = i + 1;
    if (j >= ops.size() || plans[i].role != 2 || plans[j].role != 0 || plans[j].splitk2 ||
        KERNEL_SPECS[plans[i].kernel].is_gemv())
      return false;
    const KernelSpec &s = KERNEL_SPECS[plans[j].kernel];
    if ((s.kind != KernelKind::GemmF16Mfma && s.kind != KernelKind::GemmF16Sk) ||
        !gemm_lds_ok(res[j]))
      return false;
    const Tensor *c = ops[i].call.c, *a = ops[j].call.a;
    const uint64_t a_elems = (res[j].batch_stride_a ? (uint64_t)res[j].batch : 1) * res[j].m * res[j].k;
    return a->buffer_id() == c->buffer_id() && a->device_ptr() == c->device_ptr() &&
           a_elems == (uint64_t)res[i].batch * res[i].m * res[i].n;
  }

  // `up` set: dual SwiGLU launch (ta_gemm_h16dual_*) computing `up`
  // (plain) and `op` (gate with activation and Mul{d = up.C}) in one pass.
  void launch_gemm(const KernelSpec &s, const ResolvedMatmul &d, const MatmulOp &op,
                   uint32_t splits, Scratch &scratch, CvtCache &cvt, hipStream_t stream,
                   const MatmulOp *up = nullptr, uint16_t *c16 = nullptr) const {
    void *splitk_scratch = scratch.splitk;
    GemmArgs a{};
    a.a = op.call.a->device_ptr();
    a.b = op.call.b->device_ptr();
    a.c = static_cast<float *>(splits > 1 ? splitk_scratch : op.call.c->device_ptr());
    a.stride_a = d.batch_stride_a;
    a.stride_b = d.batch_stride_b;
    a.stride_c = d.batch_stride_c;
    a.m = d.m;
    a.n = d.n;
    a.k = d.k;
    a.alpha = op.call.alpha;
    const uint32_t sub =
        splits > 1 ? splitk_sub_splits(ctx->cu_count(), d, splits) : 1;
    a.num_splits = std::max(1u, splits) * sub;
    a.sub_splits = sub;
    if (splits <= 1) {
      a.flags = op.call.accumulate ? TA_FLAG_ACCUMULATE : 0;
      if (op.epilogue.bias) {
        a.flags |= TA_FLAG_BIAS;
        a.bias = static_cast<const float *>(op.epilogue.bias->device_ptr());
        a.bias_batch_stride = op.epilogue.bias->shape().size() == 2 ? d.n : 0;
      }
      a.act = (uint32_t)op.epilogue.activation;
      a.binary = (uint32_t)op.epilogue.binary.kind;
      if (const Tensor *dt = op.epilogue.d_tensor())
        a.d = static_cast<const float *>(dt->device_ptr());
      a.beta = op.epilogue.binary.beta;
    }
    a.tiles_m = div_ceil(d.m, s.tile_m);
    a.tiles_n = div_ceil(d.n, s.tile_n);
    const uint64_t gz = (uint64_t)d.batch * a.num_splits;
    const uint64_t gx = (uint64_t)a.tiles_m * a.tiles_n;
    if (gz > 65535 || gx > 0x7fffffffull)
      fail("matmul grid (" + std::to_string(gx) + ", 1, " + std::to_string(gz) +
           ") exceeds the HIP launch limits");
    const bool lds = (s.kind == KernelKind::GemmF16Mfma || s.kind == KernelKind::GemmA16 ||
                      s.kind == KernelKind::GemmF16Sk) &&
                     gemm_lds_ok(d);
    if (lds && s.kind != KernelKind::GemmA16) {
      // A -> f16 (RNE) pre-pass into scratch; the GEMM then reads f16 A.
      CvtArgs cv{};
      cv.src = static_cast<const float *>(a.a);
      cv.dst = static_cast<uint16_t *>(splitk_scratch);
      cv.n = (d.batch_stride_a ? (uint64_t)d.batch : 1) * d.m * d.k;
      const uint64_t blocks = (cv.n + 8 * 256 - 1) / (8 * 256);
      if (blocks > 0x7fffffffull)
        fail("f16 conversion grid exceeds the HIP launch limits");
      const void *buf = op.call.a->buffer_id();
      if (CvtEntry *hit = cvt.find(buf, cv.src, cv.n)) {
        a.a = hit->base;
      } else {
        CvtEntry &v = cvt.victim();
        const CvtEntry &other = &v == &cvt.e[0] ? cvt.e[1] : cvt.e[0];
        const int half = other.half == 0 ? 1 : 0;
        const uint64_t half_bytes = scratch.splitk_bytes / 2 / 256 * 256;
        if (a16_bytes(d) > half_bytes)
          fail("internal: f16 copy scratch not reserved");
        cv.dst = reinterpret_cast<uint16_t *>(static_cast<char *>(splitk_scratch) + half * half_bytes);
        launch("ta_cvt_f32_f16", (uint32_t)blocks, 1, 1, 256, &cv, stream);
        cvt.put(v, CvtEntry{buf, cv.src, cv.n, cv.dst, SIZE_MAX, half});
        a.a = cv.dst;
      }
    } else if (splits > 1) {
      cvt.drop_region(); // the partial planes overwrite the f16 copies
    }
    const uint32_t lds_threads = (uint32_t)ta_h16_lds_threads((int)s.tile_m, (int)s.tile_n);
    if (s.kind == KernelKind::GemmF16Sk) {
      a.k_splits = h16sk_splits(ctx->cu_count(), d.batch, d.m, d.n, d.k, s.tile_m, s.tile_n);
      if (a.k_splits > 1) {
        const uint64_t tiles = (uint64_t)d.batch * a.tiles_m * a.tiles_n;
        if (scratch.partial_bytes < tiles * a.k_splits * s.tile_m * s.tile_n * 4 ||
            scratch.counters_len < tiles * TA_GEMV_COUNTER_STRIDE)
          fail("internal: split-K f16 GEMM scratch not reserved");
        a.partial = static_cast<float *>(scratch.partial);
        a.counters = scratch.counters;
      }
      if (gz > 65535 || a.k_splits > 65535)
        fail("matmul grid exceeds the HIP launch limits");
      launch(s.symbol, (uint32_t)gx, a.k_splits, (uint32_t)gz, lds_threads, &a, stream);
      return;
    }
    if (up) {
      if (!lds || s.kind != KernelKind::GemmF16Mfma || !f16_dual_tile(s) || splits > 1)
        fail("internal: dual f16w GEMM on an unsupported route");
      a.b2 = up->call.b->device_ptr();
      a.c2 = static_cast<float *>(up->call.c->device_ptr());
      a.c16 = c16;
      std::string sym = s.symbol;
      sym.replace(0, std::strlen("ta_gemm_h16_"), "ta_gemm_h16dual_");
      launch(sym + "_lds", (uint32_t)gx, 1, (uint32_t)gz, lds_threads, &a, stream);
      return;
    }
    const bool vec = d.k % 4 == 0 && d.n % 4 == 0;
    const bool mi16 = s.kind == KernelKind::GemmF32 && f32_mi16_ok(d, s.tile_m, s.tile_n,
                                                                   a.num_splits);
    const uint32_t threads = mi16  ? mi16_threads(s.tile_m)
                             : lds ? lds_threads
                                   : gemm_threads(s);
    launch(std::string(s.symbol) + (mi16 ? "_mi16" : lds ? "_lds" : vec ? "_vec" : "_gen"),
           (uint32_t)gx, 1, (uint32_t)gz, threads, &a, stream);
    if (splits > 1) {
      SplitReduceArgs r{};
      r.scratch = static_cast<const float *>(splitk_scratch);
      r.c = static_cast<float *>(op.call.c->device_ptr());
      r.mn = (uint64_t)d.m * d.n;
      r.total = r.mn * d.batch;
      r.num_splits = a.num_splits;
      const uint64_t quads = (r.total + 3) / 4;
      r.groups = splitk_reduce_groups(ctx->cu_count(), quads, r.num_splits);
      // The op's epilogue runs once, on the finished plane sum.
      r.n = d.n;
      r.flags = op.call.accumulate ? TA_FLAG_ACCUMULATE : 0;
      if (op.epilogue.bias) {
        r.flags |= TA_FLAG_BIAS;
        r.bias = static_cast<const float *>(op.epilogue.bias->device_ptr());
        r.bias_batch_stride = op.epilogue.bias->shape().size() == 2 ? d.n : 0;
      }
      r.act = (uint32_t)op.epilogue.activation;
      r.binary = (uint32_t)op.epilogue.binary.kind;
      if (const Tensor *dt = op.epilogue.d_tensor())
        r.d = static_cast<const float *>(dt->device_ptr());
      r.beta = op.epilogue.binary.beta;
      const uint64_t per_wg = kReduceThreads / r.groups;
      const uint64_t wgs = std::min<uint64_t>((quads + per_wg - 1) / per_wg, 8ull * ctx->cu_count());
      launch("ta_splitk_reduce", (uint32_t)std::max<uint64_t>(wgs, 1), 1, 1, kReduceThreads, &r,
             stream);
    }
  }

  // `up` set: dual SwiGLU launch computing `up` (plain) and `op` (gate
  // with activation and Mul{d = up.C}) in one pass.
  // Kernel arguments of one decode-GEMV job (a standalone launch, or one
  // job of a chain launch: the same unit code reads the same fields).
  static GemvArgs gemv_args(const KernelSpec &s, const ResolvedMatmul &d, const MatmulOp &op,
                            const MatmulOp *up, const GemvPlan &g) {
    const bool dual = up != nullptr;
    GemvArgs a{};
    a.x = static_cast<const float *>(op.call.a->device_ptr());
    a.w = static_cast<const uint16_t *>(op.call.b->device_ptr());
    a.y = static_cast<float *>(op.call.c->device_ptr());
    a.rows = d.m;
    a.n = d.n;
    a.k = d.k;
    a.kchunk = g.kchunk;
    a.kchunks = g.kchunks;
    a.alpha = op.call.alpha;
    a.flags = s.packed() ? TA_GEMV_PACKED : 0;
    if (op.call.accumulate)
      a.flags |= TA_FLAG_ACCUMULATE;
    if (op.epilogue.bias) {
      a.flags |= TA_FLAG_BIAS;
      a.bias = static_cast<const float *>(op.epilogue.bias->device_ptr());
    }
    a.act = (uint32_t)op.epilogue.activation;
    if (dual) {
      a.w2 = static_cast<const uint16_t *>(up->call.b->device_ptr());
      a.y2 = static_cast<float *>(up->call.c->device_ptr());
      a.binary = TA_BIN_NONE;
    } else {
      a.binary = (uint32_t)op.epilogue.binary.kind;
      if (const Tensor *dt = op.epilogue.d_tensor())
        a.d = static_cast<const float *>(dt->device_ptr());
      a.beta = op.epilogue.binary.beta;
    }
    return a;
  }

  // Decode fusions of one GEMV job (normed A, RoPE / cache-scatter store).
  static GemvFusion gemv_fusion(const MatmulOp &op, bool dual) {
    GemvFusion fu{};
    if (op.normed_a) {
      fu.norm_w = static_cast<const float *>(op.normed_a->weight->device_ptr());
      fu.norm_eps = op.normed_a->eps;
    }
    if (!op.store.is_none()) {
      if (dual)
        fail("internal: store epilogue on a dual GEMV launch");
      const MatmulStoreDesc &sd = op.store.desc;
      fu.store_mode = op.store.mode();
      fu.head_dim = sd.head_dim;
      fu.pos_base = sd.pos_base;
      fu.pos_scale = sd.pos_scale;
      fu.stride_head = sd.stride_head;
      fu.stride_dim = sd.stride_dim;
      fu.pos_addr = reinterpret_cast<const uint32_t *>(sd.pos_addr);
      if (op.store.table) {
        fu.rope_table = static_cast<const float *>(op.store.table->device_ptr());
        fu.table_len = op.store.table->len();
      }
      if (op.store.dst) {
        fu.store_dst = op.store.dst->device_ptr();
        fu.store_dst_f16 = op.store.dst->dtype() == DType::F16 ? 1u : 0u;
        fu.dst_len = op.store.dst->len();
      }
    }
    return fu;
  }

  void launch_gemv(const KernelSpec &s, const ResolvedMatmul &d, const MatmulOp &op,
                   const MatmulOp *up, Scratch &scratch, hipStream_t stream) const {
    const bool dual = up != nullptr;
    GemvPlan g = plan_gemv(ctx->cu_count(), d.m, d.n, d.k, s.tile_n, dual,
                          gemv_unit(s.tile_n, s.kind == KernelKind::GemvF32Row, dual, d.m));
    GemvArgs a = gemv_args(s, d, op, up, g);
    if (g.kchunks > 1) {
      if (scratch.partial_bytes < g.partial_bytes || scratch.counters_len < (uint64_t)g.tiles * TA_GEMV_COUNTER_STRIDE)
        fail("internal: GEMV scratch not reserved");
      a.partial = static_cast<float *>(scratch.partial);
      a.counters = scratch.counters;
    }
    GemvFusion fu = gemv_fusion(op, dual);
    std::string sym = std::string(s.symbol) + (dual ? "_dual" : "") + "_m" + std::to_string(g.mr);
    launch(sym, g.tiles * g.kchunks, 1, 1, 256, &a, stream, &fu);
  }

  // Dual SwiGLU fusion in a dependent graph: op i = x @ Wu (plain) and op
  // i+1 = act(x @ Wg [+ bias]) * C_i on the same decode GEMV route become
  // one launch that streams Wg and Wu together and writes both outputs.
  // Same route for both ops: the decode GEMV (dual launch) or the
  // pipelined f16w GEMM on a tile with a dual kernel (ta_gemm_h16dual_*).
  static bool fusable_pair(const MatmulOp &up, const OpPlan &pu, const MatmulOp &gate,
                           const OpPlan &pg, const ResolvedMatmul &d) {
    if (pu.kernel != pg.kernel || !KERNEL_SPECS[pu.kernel].weights_f16() || pu.splitk2 ||
        pg.splitk2)
      return false;
    const KernelSpec &s = KERNEL_SPECS[pu.kernel];
    if (!s.is_gemv() && !(f16_dual_tile(s) && gemm_lds_ok(d)))
      return false;
    if (!up.epilogue.is_none() || up.call.accumulate || gate.call.accumulate ||
        !up.store.is_none() || !gate.store.is_none())
      return false;
    // Normed A (RMSNorm folded into the GEMV's X staging): the same norm on
    // both, and only on the decode GEMV, whose dual unit applies it.
    if (up.normed_a.has_value() != gate.normed_a.has_value())
      return false;
    if (up.normed_a &&
        (!s.is_gemv() || up.normed_a->weight->buffer_id() != gate.normed_a->weight->buffer_id() ||
         up.normed_a->eps != gate.normed_a->eps))
      return false;
    if (gate.epilogue.binary.kind != EpilogueBinary::Kind::Mul ||
        gate.epilogue.binary.d->buffer_id() != up.call.c->buffer_id())
      return false;
    if (gate.epilogue.bias && (gate.epilogue.bias->buffer_id() == up.call.c->buffer_id() ||
                               gate.epilogue.bias->shape().size() != 1))
      return false;
    if (up.call.a->buffer_id() != gate.call.a->buffer_id() ||
        up.call.a->shape() != gate.call.a->shape() || up.call.b->shape() != gate.call.b->shape() ||
        up.call.c->shape() != gate.call.c->shape() || up.call.alpha != gate.call.alpha ||
        up.packed_b != gate.packed_b || up.call.b->dtype() != gate.call.b->dtype())
      return false;
    return gate.call.c->buffer_id() != up.call.c->buffer_id();
  }

  void mark_fusions(const std::vector<MatmulOp> &ops, const std::vector<ResolvedMatmul> &res,
                    std::vector<OpPlan> &plans) const {
    if (std::getenv("TA_NO_FUSE"))
      return;
    for (size_t i = 0; i + 1 < ops.size(); ++i) {
      if (plans[i].role != 0 || plans[i + 1].role != 0)
        continue;
      if (!std::getenv("TA_NO_MLP") && i + 2 < ops.size() && plans[i + 2].role == 0 &&
          res[i].batch == 1 && res[i].m <= mlp_max_rows() &&
          fusable_pair(ops[i], plans[i], ops[i + 1], plans[i + 1], res[i]) &&
          mlp_tail_ok(ops[i], ops[i + 1], plans[i + 1], ops[i + 2], plans[i + 2])) {
        plans[i].role = 3;
        plans[i].mlp_layers = 1;
        plans[i + 1].role = 4;
        plans[i + 2].role = 4;
        i += 2;
        continue;
      }
      if (fusable_pair(ops[i], plans[i], ops[i + 1], plans[i + 1], res[i])) {
        plans[i].role = 1;
        plans[i + 1].role = 2;
        ++i;
      }
    }
    if (std::getenv("TA_NO_MLP_CHAIN"))
      return;
    // Decode-MLP chains: consecutive MLP launches where each reads the
    // previous one's output as x become one launch.
    for (size_t i = 0; i < ops.size(); ++i) {
      if (plans[i].role != 3)
        continue;
      size_t j = i + 3;
      while (plans[i].mlp_layers < TA_MLP_MAX_LAYERS && j < ops.size() && plans[j].role == 3 &&
             mlp_chain_ok(ops, res, i, j)) {
        plans[j].role = 4;
        plans[j].mlp_layers = 0;
        ++plans[i].mlp_layers;
        j += 3;
      }
      i = j - 1;
    }
  }

  // Rows up to which op triples become decode-MLP launches: every M the
  // kernels have (1..8; from 4 rows the inner product runs on the matrix
  // cores and the hand-offs pre-poll sentinels, which made the chain
  // faster than the separate dual gate/up and down launches at M = 4 and
  // 8 as well).  TA_MLP_MAX_ROWS lowers it (at most 8).
  static uint32_t mlp_max_rows() {
    uint32_t rows = 8;
    if (const char *env = std::getenv("TA_MLP_MAX_ROWS"))
      rows = (uint32_t)std::strtoul(env, nullptr, 10);
    return std::min<uint32_t>(rows, 8);
  }

  // May the MLP at ops[j..j+2] join the chain that starts at ops[i] and
  // ends just before j?  Same shapes; its x is the previous layer's y (read
  // through the tagged hand-off); its biases, read with plain loads, are
  // not written by the chain.  Every other buffer is safe: chained layers
  // write their outputs with agent-scope stores, read the residual with
  // agent-scope loads, and run after every earlier layer has finished.
  static bool mlp_chain_ok(const std::vector<MatmulOp> &ops,
                           const std::vector<ResolvedMatmul> &res, size_t i, size_t j) {
    for (size_t k = 0; k < 3; ++k)
      if (res[j + k].m != res[i + k].m || res[j + k].n != res[i + k].n ||
          res[j + k].k != res[i + k].k)
        return false;
    // A later layer's x is the previous layer's y, handed over inside the
    // launch: it cannot be normed (its norm needs the whole row first).
    if (ops[j].normed_a)
      return false;
    const Tensor *prev_y = ops[j - 1].call.c, *x = ops[j].call.a;
    if (x->buffer_id() != prev_y->buffer_id() || x->shape() != prev_y->shape() ||
        ops[j + 1].call.a->buffer_id() != x->buffer_id())
      return false;
    for (const Tensor *bias : {ops[j + 1].epilogue.bias, ops[j + 2].epilogue.bias}) {
      if (!bias)
        continue;
      for (size_t k = i; k < j; ++k)
        if (bias->buffer_id() == ops[k].call.c->buffer_id())
          return false;
    }
    return true;
  }

  // src/executor/recording.rs:204-235: a route without the fused
  // normed-A / store body fails instead of silently skipping it.
  static void check_fusions(const KernelSpec &s, const MatmulOp &op, const ResolvedMatmul &d) {
    if (op.normed_a && !s.supports_normed_a())
      fail(std::string("kernel '") + s.name +
           "' does not implement the fused normed-A GEMV (decode GEMV kernels only; normed-A "
           "requires a decode GEMV route with M <= 8 and batch 1, got M=" +
           std::to_string(d.m) + ")");
    if (!op.store.is_none() && !s.supports_store())
      fail(std::string("kernel '") + s.name +
           "' does not implement the fused store epilogue (f16-weight decode GEMV kernels "
           "only; store requires an M=1 f16-weights GEMV route, got M=" +
           std::to_string(d.m) + ")");
  }

  void check_supported(const KernelSpec &s, const ResolvedMatmul &d) const {
    if (!kernel_supports(s, d)) {
      std::ostringstream o;
      o << "kernel '" << s.name << "' cannot run B=" << d.batch << " " << d.m << "x" << d.n
        << "x" << d.k << (d.b_f16 ? " (f16 B)" : " (f32 B)") << (d.packed_b ? " packed" : "");
      fail(o.str());
    }
  }

  ScratchNeed total_need(const std::vector<ResolvedMatmul> &res,
                         const std::vector<OpPlan> &plans) const {
    ScratchNeed need;
    for (size_t i = 0; i < res.size(); ++i) {
      if (plans[i].role == 3) {
        MlpGeom g = mlp_geom(res[i], res[i + 2]);
        ScratchNeed m;
        m.mlp = g.bytes;
        need.merge(m);
      } else if (plans[i].role == 5) {
        const ChainGeom g = chain_geom(res, i, plans[i].chain_jobs);
        ScratchNeed c;
        c.partial = g.partial_bytes;
        c.counters = g.counters;
        c.barrier = true;
        need.merge(c);
      } else if (plans[i].role == 6) {
        continue;
      } else if (plans[i].role != 1 && plans[i].role != 4) {
        need.merge(scratch_need(res[i], plans[i]));
        if (plans[i].role == 2 && !KERNEL_SPECS[plans[i].kernel].is_gemv()) {
          ScratchNeed c; // f16 copy of a dual launch's output (f16_copy_feeds_next)
          c.shadow = (uint64_t)res[i].batch * res[i].m * res[i].n * 2;
          need.merge(c);
        }
      }
    }
    return need;
  }

  // ---- persistent decode MLP: [up, gate*act*up, down] in one launch ----
  // Byte offsets into Scratch::mlp: generation word, done counter (own
  // 128-byte lines), then the tagged words of the gate/up partials, of h
  // and of the down partials.
  struct MlpGeom {
    uint32_t mr, tiles_a, kch_a, tiles_b, kch_b;
    uint64_t gen, done, tag_a, tag_h, tag_b, tag_y, bytes;
  };
  // K windows of the two phases (shared with the kernel).
  static constexpr uint32_t kMlpRowsA = TA_MLP_ROWS_A, kMlpRowsB = TA_MLP_ROWS_B;

  static MlpGeom mlp_geom(const ResolvedMatmul &up, const ResolvedMatmul &down) {
    MlpGeom g{};
    g.mr = up.m <= 1 ? 1 : up.m <= 2 ? 2 : up.m <= 4 ? 4 : 8;
    g.tiles_a = up.n / 64;
    g.kch_a = (up.k + kMlpRowsA - 1) / kMlpRowsA;
    g.tiles_b = down.n / 64;
    g.kch_b = (down.k + kMlpRowsB - 1) / kMlpRowsB;
    auto al = [](uint64_t v) { return (v + 255) / 256 * 256; };
    g.gen = 0;
    g.done = 128;
    g.tag_a = 256;
    g.tag_h = al(g.tag_a + (uint64_t)g.kch_a * g.tiles_a * 2 * g.mr * 64 * 8);
    g.tag_b = al(g.tag_h + (uint64_t)down.k * g.mr * 8);
    g.tag_y = al(g.tag_b + (uint64_t)g.kch_b * g.tiles_b * g.mr * 64 * 8);
    g.bytes = al(g.tag_y + (uint64_t)down.n * g.mr * 8);
    return g;
  }

  // ops[i] = x@Wu, ops[i+1] = act(x@Wg) * up (a fusable pair), ops[i+2] =
  // h@Wd reading the pair's output h, all on the packed 64-column decode
  // GEMV.  The down op keeps its full epilogue.  Its output may not be a
  // buffer the pair writes (plain and agent-scope stores would race) or
  // reads as x; its bias (plain loads) and residual may not be a pair
  // output.
  static bool mlp_tail_ok(const MatmulOp &up, const MatmulOp &gate, const OpPlan &pg,
                          const MatmulOp &down, const OpPlan &pd) {
    const KernelSpec &sg = KERNEL_SPECS[pg.kernel], &sd = KERNEL_SPECS[pd.kernel];
    if (!sg.packed() || !sd.packed() || sg.tile_n != 64 || sd.tile_n != 64 || pd.splitk2)
      return false;
    // Whole K windows in both phases (the kernel does not mask rows).
    if (gate.call.a->shape().back() % kMlpRowsA != 0 || down.call.a->shape().back() % kMlpRowsB != 0)
      return false;
    if (down.has_decode_fusion())
      return false;
    if (!down.packed_b || down.call.a->buffer_id() != gate.call.c->buffer_id() ||
        down.call.a->shape() != gate.call.c->shape())
      return false;
    auto pair_out = [&](const Tensor *t) {
      return t && (t->buffer_id() == up.call.c->buffer_id() ||
                   t->buffer_id() == gate.call.c->buffer_id());
    };
    return !pair_out(down.call.c) && down.call.c->buffer_id() != up.call.a->buffer_id() &&
           !pair_out(down.epilogue.bias) && !pair_out(down.epilogue.d_tensor());
  }

  // Decode-MLP chain of `layers` layers starting at ops[i] (each layer is
  // the op triple [up, gate, down]).
  void launch_mlp(const std::vector<MatmulOp> &ops, const std::vector<ResolvedMatmul> &res,
                  size_t i, uint32_t layers, Scratch &scratch, uint32_t *host_status,
                  hipStream_t stream) const {
    MlpGeom g = mlp_geom(res[i], res[i + 2]);
    if (scratch.mlp_bytes < g.bytes)
      fail("internal: decode-MLP scratch not reserved");
    if (!host_status)
      fail("internal: decode-MLP status word missing");
    if (layers < 1 || layers > TA_MLP_MAX_LAYERS || i + 3 * layers > ops.size())
      fail("internal: bad decode-MLP chain length");
    MlpArgs m{};
    if (ops[i].normed_a) {
      m.norm_w = static_cast<const float *>(ops[i].normed_a->weight->device_ptr());
      m.norm_eps = ops[i].normed_a->eps;
    }
    for (uint32_t l = 0; l < layers; ++l) {
      const size_t o = i + 3 * (size_t)l;
      const MatmulOp &up = ops[o], &gate = ops[o + 1], &down = ops[o + 2];
      GemvArgs &a = m.layer[l].a;
      a.x = static_cast<const float *>(gate.call.a->device_ptr());
      a.w = static_cast<const uint16_t *>(gate.call.b->device_ptr());
      a.w2 = static_cast<const uint16_t *>(up.call.b->device_ptr());
      a.y = static_cast<float *>(gate.call.c->device_ptr());
      a.y2 = static_cast<float *>(up.call.c->device_ptr());
      a.rows = res[o].m;
      a.n = res[o].n;
      a.k = res[o].k;
      a.kchunk = kMlpRowsA;
      a.kchunks = g.kch_a;
      a.flags = TA_GEMV_PACKED;
      if (gate.epilogue.bias) {
        a.flags |= TA_FLAG_BIAS;
        a.bias = static_cast<const float *>(gate.epilogue.bias->device_ptr());
      }
      a.act = (uint32_t)gate.epilogue.activation;
      a.alpha = gate.call.alpha;
      GemvArgs &b = m.layer[l].b;
      b.x = static_cast<const float *>(down.call.a->device_ptr());
      b.w = static_cast<const uint16_t *>(down.call.b->device_ptr());
      b.y = static_cast<float *>(down.call.c->device_ptr());
      b.rows = res[o + 2].m;
      b.n = res[o + 2].n;
      b.k = res[o + 2].k;
      b.kchunk = kMlpRowsB;
      b.kchunks = g.kch_b;
      b.flags = TA_GEMV_PACKED | (down.call.accumulate ? TA_FLAG_ACCUMULATE : 0u);
      if (down.epilogue.bias) {
        b.flags |= TA_FLAG_BIAS;
        b.bias = static_cast<const float *>(down.epilogue.bias->device_ptr());
      }
      b.act = (uint32_t)down.epilogue.activation;
      b.binary = (uint32_t)down.epilogue.binary.kind;
      if (const Tensor *dt = down.epilogue.d_tensor())
        b.d = static_cast<const float *>(dt->device_ptr());
      b.beta = down.epilogue.binary.beta;
      b.alpha = down.call.alpha;
    }
    char *base = static_cast<char *>(scratch.mlp);
    m.gen = reinterpret_cast<uint32_t *>(base + g.gen);
    m.done = reinterpret_cast<uint32_t *>(base + g.done);
    m.tag_a = reinterpret_cast<uint64_t *>(base + g.tag_a);
    m.tag_h = reinterpret_cast<uint64_t *>(base + g.tag_h);
    m.tag_b = reinterpret_cast<uint64_t *>(base + g.tag_b);
    m.tag_y = reinterpret_cast<uint64_t *>(base + g.tag_y);
    m.spin_limit = 1u << 20; // ~1 s of polling (a round is about a memory round trip)
    void *dev_status = device_status(host_status);
    m.status = static_cast<uint32_t *>(dev_status);
    m.units_a = g.tiles_a * g.kch_a;
    m.units_b = g.tiles_b * g.kch_b;
    m.tiles_a = g.tiles_a;
    m.tiles_b = g.tiles_b;
    m.layers = layers;
    launch("ta_decode_mlp_f16_t64_m" + std::to_string(g.mr), layers * (m.units_a + m.units_b), 1,
           1, 256, &m, stream);
  }

  // ---- persistent GEMV chain (src/executor/elementwise/gemv_chain.rs) ----
  // Each job keeps the K windows its standalone row-GEMV launch would take
  // (the same plan_gemv call), so its units, window reduction and epilogue
  // are that launch's; the jobs' partial planes and tile counters sit end
  // to end in the scratch regions.
  struct ChainGeom {
    std::vector<GemvPlan> plans;
    std::vector<uint64_t> partial_off, counter_off;
    uint64_t partial_bytes = 0, counters = 0;
  };
  ChainGeom chain_geom(const std::vector<ResolvedMatmul> &res, size_t i, uint32_t n) const {
    ChainGeom g;
    for (size_t j = i; j < i + n; ++j) {
      const ResolvedMatmul &d = res[j];
      g.plans.push_back(plan_gemv(ctx->cu_count(), d.m, d.n, d.k, 64, false,
                                  gemv_unit(64, false, false, d.m)));
      g.partial_off.push_back(g.partial_bytes);
      g.counter_off.push_back(g.counters);
      g.partial_bytes += (g.plans.back().partial_bytes + 255) / 256 * 256;
      g.counters += (uint64_t)g.plans.back().tiles * TA_GEMV_COUNTER_STRIDE;
    }
    return g;
  }

  // gemv_chain.rs:200-240 (gemv_jobs_hazard): does job `next` read what an
  // earlier job of the chain writes, or write what one reads or writes?
  static bool chain_hazard(const std::vector<MatmulOp> &ops, size_t first, size_t next) {
    auto reads = [](const MatmulOp &op) {
      std::vector<const void *> v{op.call.a->buffer_id(), op.call.b->buffer_id()};
      if (const Tensor *d = op.epilogue.d_tensor())
        v.push_back(d->buffer_id());
      if (op.normed_a)
        v.push_back(op.normed_a->weight->buffer_id());
      if (op.call.accumulate)
        v.push_back(op.call.c->buffer_id());
      if (op.epilogue.bias)
        v.push_back(op.epilogue.bias->buffer_id());
      if (op.store.table)
        v.push_back(op.store.table->buffer_id());
      return v;
    };
    // Outputs: C, and a store epilogue's destination (the KV cache).
    auto writes = [](const MatmulOp &op) {
      std::vector<const void *> v{op.call.c->buffer_id()};
      if (op.store.dst)
        v.push_back(op.store.dst->buffer_id());
      return v;
    };
    auto meets = [](const std::vector<const void *> &a, const std::vector<const void *> &b) {
      for (const void *x : a)
        if (std::find(b.begin(), b.end(), x) != b.end())
          return true;
      return false;
    };
    const auto next_reads = reads(ops[next]), next_writes = writes(ops[next]);
    for (size_t j = first; j < next; ++j) {
      const auto prev_writes = writes(ops[j]);
      if (meets(next_reads, prev_writes) || meets(next_writes, prev_writes) ||
          meets(next_writes, reads(ops[j])))
        return true;
    }
    return false;
  }

  // Roles of a GEMV chain's ops: one persistent launch when it is enabled
  // (ML_DEVICE_SCOPE=1, the reference's opt-in for its persistent chain,
  // src/context/init.rs:292-307) and every job takes the row-major f16
  // decode GEMV (M = 1, N % 4 == 0); otherwise the jobs run as separate
  // launches in list order (with the graph fusions), which measured faster
  // on this chip (a 7-job decode chain: 69 us against 78 us).  Both give
  // the same bits.
  static bool chain_enabled() {
    const char *v = std::getenv("ML_DEVICE_SCOPE");
    if (!v)
      return false;
    std::string t(v);
    for (char &ch : t)
      ch = (char)std::tolower((unsigned char)ch);
    return t == "1" || t == "true";
  }
  static bool mark_chain(const std::vector<ResolvedMatmul> &res, std::vector<OpPlan> &plans) {
    if (!chain_enabled() || plans.empty() || plans.size() > TA_GEMV_CHAIN_MAX_JOBS)
      return false;
    for (size_t j = 0; j < plans.size(); ++j)
      if (KERNEL_SPECS[plans[j].kernel].kind != KernelKind::GemvF16Row || plans[j].splitk2 ||
          res[j].m != 1 || res[j].batch != 1)
        return false;
    plans[0].role = 5;
    plans[0].chain_jobs = (uint32_t)plans.size();
    for (size_t j = 1; j < plans.size(); ++j)
      plans[j].role = 6;
    return true;
  }

  // GEMV groups: consecutive one-row f16 decode GEMVs (64-column tiles,
  // row-major or packed) that do not touch each other's data run as one
  // chain launch with no barrier: their units share one grid, so small
  // jobs such as the q, k and v projections fill the CUs together instead
  // of one launch each (TinyLlama q/k/v with normed A: 13.4 us against
  // 27.2 us as three launches).  A job reads and writes what its own
  // launch would, through the same unit code, so the results are the same
  // bits.  Launches between groups stay kernel boundaries.
  // TA_NO_GEMV_GROUP keeps one launch per job (route control).
  static bool groupable(const OpPlan &p, const ResolvedMatmul &d) {
    const KernelSpec &s = KERNEL_SPECS[p.kernel];
    return p.role == 0 && !p.splitk2 && s.tile_n == 64 &&
           (s.kind == KernelKind::GemvF16Row || s.kind == KernelKind::GemvF16Packed) &&
           d.m == 1 && d.batch == 1;
  }
  static void mark_groups(const std::vector<MatmulOp> &ops, const std::vector<ResolvedMatmul> &res,
                          std::vector<OpPlan> &plans) {
    if (std::getenv("TA_NO_GEMV_GROUP"))
      return;
    for (size_t i = 0; i < ops.size();) {
      size_t j = i;
      while (groupable(plans[j], res[j]) && j + 1 < ops.size() &&
             j + 1 - i < TA_GEMV_CHAIN_MAX_JOBS && groupable(plans[j + 1], res[j + 1]) &&
             !chain_hazard(ops, i, j + 1))
        ++j;
      if (j > i) {
        plans[i].role = 5;
        plans[i].chain_jobs = (uint32_t)(j - i + 1);
        for (size_t q = i + 1; q <= j; ++q)
          plans[q].role = 6;
      }
      i = j + 1;
    }
  }

  void launch_chain(const std::vector<MatmulOp> &ops, const std::vector<ResolvedMatmul> &res,
                    const std::vector<OpPlan> &plans, size_t i, uint32_t n, Scratch &scratch,
                    uint32_t *host_status, hipStream_t stream) const {
    if (n < 1 || n > TA_GEMV_CHAIN_MAX_JOBS || i + n > ops.size())
      fail("internal: bad GEMV chain length");
    const ChainGeom g = chain_geom(res, i, n);
    if (scratch.partial_bytes < g.partial_bytes || scratch.counters_len < g.counters ||
        !scratch.barrier)
      fail("internal: GEMV chain scratch not reserved");
    if (!host_status)
      fail("internal: GEMV chain status word missing");
    GemvChainArgs c{};
    for (uint32_t j = 0; j < n; ++j) {
      const MatmulOp &op = ops[i + j];
      const GemvPlan &gp = g.plans[j];
      GemvArgs &a = c.job[j];
      a = gemv_args(KERNEL_SPECS[plans[i + j].kernel], res[i + j], op, nullptr, gp);
      if (gp.kchunks > 1) {
        a.partial = reinterpret_cast<float *>(static_cast<char *>(scratch.partial) + g.partial_off[j]);
        a.counters = scratch.counters + g.counter_off[j];
      }
      c.fu[j] = gemv_fusion(op, false);
      c.units[j] = gp.tiles * gp.kchunks;
      if (j + 1 < n && chain_hazard(ops, i, i + j + 1))
        c.sync_after |= 1u << j;
    }
    uint64_t widest = 0, group = 0;
    for (uint32_t j = 0; j < n; ++j) {
      group += c.units[j];
      if (j + 1 == n || ((c.sync_after >> j) & 1u)) {
        widest = std::max(widest, group);
        group = 0;
      }
    }
    c.n_jobs = n;
    c.spin_limit = 1u << 22; // ~seconds of polling: a safety net, see the kernel
    c.barrier = scratch.barrier;
    void *dev_status = device_status(host_status);
    c.status = static_cast<uint32_t *>(dev_status);
    const uint64_t grid = std::max<uint64_t>(1, std::min<uint64_t>(widest, 2ull * ctx->cu_count()));
    launch("ta_gemv_chain_f16_m1", (uint32_t)grid, 1, 1, 256, &c, stream);
  }

  // run_gemv_chain (gemv_chain.rs:181-193): one persistent launch.
  RunStats run_chain_impl(const std::vector<MatmulOp> &jobs) {
    ctx->make_current();
    for (const auto &op : jobs)
      validate_op(op);
    std::vector<ResolvedMatmul> res;
    for (const auto &op : jobs)
      res.push_back(ResolvedMatmul::from_op(op));
    std::vector<OpPlan> plans;
    for (size_t i = 0; i < jobs.size(); ++i)
      plans.push_back(plan_op(jobs[i], res[i], false));
    if (!mark_chain(res, plans)) {
      mark_fusions(jobs, res, plans);
      mark_groups(jobs, res, plans);
    }
    Lease lease(this);
    const uint64_t ns = submit_and_wait(lease.s, jobs, res, plans);
    return RunStats{ns, jobs.size(), total_flops(res)};
  }

  // Launches that report through the host status word: the decode MLP
  // and the persistent GEMV chain.
  static bool has_mlp(const std::vector<OpPlan> &plans) {
    for (const auto &p : plans)
      if (p.role == 3 || p.role == 5)
        return true;
    return false;
  }

  void record(const std::vector<MatmulOp> &ops, const std::vector<ResolvedMatmul> &res,
              const std::vector<OpPlan> &plans, Scratch &scratch, uint32_t *host_status,
              hipStream_t stream) const {
    CvtCache cvt;
    convert_inputs_up_front(ops, res, plans, scratch, cvt, stream);
    for (size_t i = 0; i < ops.size(); ++i) {
      const OpPlan &p = plans[i];
      // a cached f16 copy of A is stale once an op writes A's buffer
      // (except the op whose epilogue wrote the copy)
      if (i > 0) {
        cvt.wrote(ops[i - 1].call.c->buffer_id(), i - 1);
        if (ops[i - 1].store.dst)
          cvt.wrote(ops[i - 1].store.dst->buffer_id(), i - 1);
      }
      if (p.role == 1 || p.role == 4 || p.role == 6)
        continue; // produced by the dual launch of op i+1 / the MLP / chain launch
      if (p.role == 5) {
        for (size_t j = i; j < i + p.chain_jobs; ++j) {
          check_supported(KERNEL_SPECS[plans[j].kernel], res[j]);
          check_fusions(KERNEL_SPECS[plans[j].kernel], ops[j], res[j]);
        }
        launch_chain(ops, res, plans, i, p.chain_jobs, scratch, host_status, stream);
        continue;
      }
      if (p.role == 3) {
        for (size_t j = i; j < i + 3 * (size_t)p.mlp_layers; ++j)
          check_supported(KERNEL_SPECS[plans[j].kernel], res[j]);
        launch_mlp(ops, res, i, p.mlp_layers, scratch, host_status, stream);
        continue;
      }
      const KernelSpec &s = KERNEL_SPECS[p.kernel];
      check_supported(s, res[i]);
      check_fusions(s, ops[i], res[i]);
      if (s.is_gemv())
        launch_gemv(s, res[i], ops[i], p.role == 2 ? &ops[i - 1] : nullptr, scratch, stream);
      else if (p.role == 2 && f16_copy_feeds_next(ops, res, plans, i)) {
        if (scratch.shadow_bytes < (uint64_t)res[i].batch * res[i].m * res[i].n * 2)
          fail("internal: f16 output copy scratch not reserved");
        uint16_t *c16 = static_cast<uint16_t *>(scratch.shadow);
        launch_gemm(s, res[i], ops[i], 1, scratch, cvt, stream, &ops[i - 1], c16);
        cvt.wrote(ops[i].call.c->buffer_id(), SIZE_MAX);
        cvt.put(cvt.victim(), CvtEntry{ops[i].call.c->buffer_id(), ops[i].call.c->device_ptr(),
                                       (uint64_t)res[i].batch * res[i].m * res[i].n, c16, i, -1});
      } else
        launch_gemm(s, res[i], ops[i], p.splitk2.value_or(1), scratch, cvt, stream,
                    p.role == 2 ? &ops[i - 1] : nullptr);
    }
  }

  // Submit `ops` on a slot and wait; returns GPU ns between the events.
  uint64_t submit_and_wait(Slot *slot, const std::vector<MatmulOp> &ops,
                           const std::vector<ResolvedMatmul> &res,
                           const std::vector<OpPlan> &plans) const {
    ScratchNeed need = total_need(res, plans);
    slot->scratch.ensure(need.splitk, need.partial, need.counters);
    slot->scratch.ensure_mlp(need.mlp);
    slot->scratch.ensure_shadow(need.shadow);
    slot->scratch.ensure_barrier(need.barrier);
    return submit_on(slot, ops, res, plans, slot->scratch);
  }
  // run_ops with several independent ops (src/executor/dispatch.rs:55-60:
  // no barriers between them): ops are spread over the slot's stream and
  // its side lanes (largest first, each to the lane with the least work so
  // far, in a deterministic order), forked from and joined back into the
  // slot's stream with events.  Each lane has its own scratch; an op's
  // result does not depend on the lane it ran on.
  uint64_t submit_concurrent(Slot *slot, const std::vector<MatmulOp> &ops,
                             const std::vector<ResolvedMatmul> &res,
                             const std::vector<OpPlan> &plans) const {
    const size_t lanes = std::min(kRunOpsLanes, ops.size());
    if (slot->side.size() + 1 < lanes) {
      if (!slot->fork)
        hip_check(hipEventCreateWithFlags(&slot->fork, hipEventDisableTiming), "hipEventCreate");
      while (slot->side.size() + 1 < lanes) {
        SideLane l;
        hip_check(hipStreamCreateWithFlags(&l.stream, hipStreamNonBlocking), "hipStreamCreate");
        hip_check(hipEventCreateWithFlags(&l.done, hipEventDisableTiming), "hipEventCreate");
        slot->side.push_back(std::move(l));
      }
    }
    std::vector<size_t> order(ops.size());
    for (size_t i = 0; i < order.size(); ++i)
      order[i] = i;
    std::stable_sort(order.begin(), order.end(), [&](size_t x, size_t y) {
      return res[x].total_flops > res[y].total_flops;
    });
    std::vector<uint64_t> load(lanes, 0);
    std::vector<std::vector<size_t>> members(lanes);
    for (size_t i : order) {
      const size_t l = std::min_element(load.begin(), load.end()) - load.begin();
      load[l] += std::max<uint64_t>(res[i].total_flops, 1);
      members[l].push_back(i);
    }
    struct Part {
      std::vector<MatmulOp> ops;
      std::vector<ResolvedMatmul> res;
      std::vector<OpPlan> plans;
    };
    std::vector<Part> parts(lanes);
    for (size_t l = 0; l < lanes; ++l) {
      std::sort(members[l].begin(), members[l].end());
      for (size_t i : members[l]) {
        parts[l].ops.push_back(ops[i]);
        parts[l].res.push_back(res[i]);
        parts[l].plans.push_back(plans[i]);
      }
      const ScratchNeed need = total_need(parts[l].res, parts[l].plans);
      Scratch &sc = l == 0 ? slot->scratch : slot->side[l - 1].scratch;
      sc.ensure(need.splitk, need.partial, need.counters);
      sc.ensure_mlp(need.mlp);
      sc.ensure_shadow(need.shadow);
      sc.ensure_barrier(need.barrier);
    }
    hip_check(hipEventRecord(slot->start, slot->stream), "hipEventRecord");
    hip_check(hipEventRecord(slot->fork, slot->stream), "hipEventRecord");
    for (size_t l = 1; l < lanes; ++l)
      hip_check(hipStreamWaitEvent(slot->side[l - 1].stream, slot->fork, 0), "hipStreamWaitEvent");
    for (size_t l = 0; l < lanes; ++l) {
      hipStream_t st = l == 0 ? slot->stream : slot->side[l - 1].stream;
      Scratch &sc = l == 0 ? slot->scratch : slot->side[l - 1].scratch;
      record(parts[l].ops, parts[l].res, parts[l].plans, sc, slot->host_status, st);
    }
    for (size_t l = 1; l < lanes; ++l) {
      hip_check(hipEventRecord(slot->side[l - 1].done, slot->side[l - 1].stream), "hipEventRecord");
      hip_check(hipStreamWaitEvent(slot->stream, slot->side[l - 1].done, 0), "hipStreamWaitEvent");
    }
    hip_check(hipEventRecord(slot->end, slot->stream), "hipEventRecord");
    hip_check(hipEventSynchronize(slot->end), "hipEventSynchronize");
    float ms = 0.f;
    hip_check(hipEventElapsedTime(&ms, slot->start, slot->end), "hipEventElapsedTime");
    return (uint64_t)((double)ms * 1e6);
  }

  // Submit with the given scratch, which already holds what the plans need.
  uint64_t submit_on(Slot *slot, const std::vector<MatmulOp> &ops,
                     const std::vector<ResolvedMatmul> &res, const std::vector<OpPlan> &plans,
                     Scratch &scratch) const {
    hip_check(hipEventRecord(slot->start, slot->stream), "hipEventRecord");
    record(ops, res, plans, scratch, slot->host_status, slot->stream);
    hip_check(hipEventRecord(slot->end, slot->stream), "hipEventRecord");
    hip_check(hipEventSynchronize(slot->end), "hipEventSynchronize");
    float ms = 0.f;
    hip_check(hipEventElapsedTime(&ms, slot->start, slot->end), "hipEventElapsedTime");
    if (has_mlp(plans))
      check_host_status(slot->host_status, scratch.mlp, scratch.mlp_bytes);
    return (uint64_t)((double)ms * 1e6);
  }

  // One model-op launch on a slot between its events
  // (elementwise/mod.rs:498-515: n_calls 1, no flops).
  RunStats run_elem(const ElemLaunch &l) { return run_elem(ElemLaunches{l}); }
  RunStats run_elem(const ElemLaunches &ls) {
    ctx->make_current();
    Lease lease(this);
    Slot *slot = lease.s;
    hip_check(hipEventRecord(slot->start, slot->stream), "hipEventRecord");
    record_elem(ls, slot->stream);
    hip_check(hipEventRecord(slot->end, slot->stream), "hipEventRecord");
    hip_check(hipEventSynchronize(slot->end), "hipEventSynchronize");
    float ms = 0.f;
    hip_check(hipEventElapsedTime(&ms, slot->start, slot->end), "hipEventElapsedTime");
    return RunStats{(uint64_t)((double)ms * 1e6), ls.size(), 0};
  }
  void record_elem(const ElemLaunches &ls, hipStream_t stream) const {
    for (const ElemLaunch &l : ls)
      launch(l.symbol, l.groups, l.gy, 1, l.threads, const_cast<uint8_t *>(l.args.data()),
             stream);
  }

  // ---- mixed-op graphs (src/executor/graph_ops.rs:244-620) ----
  // Consecutive matmuls form one segment, routed like run_op_graph (pair
  // and decode-MLP fusion stay inside a segment); each model op is one
  // launch.  Stream order provides every op's dependency on earlier ones.
  struct ExecStep {
    bool matmul = false;
    bool chain = false; // a GEMV chain's jobs (one persistent launch when eligible)
    std::vector<MatmulOp> ops;
    std::vector<ResolvedMatmul> res;
    std::vector<OpPlan> plans;
    ElemLaunches elems;
  };
  std::vector<ExecStep> plan_exec(const std::vector<ExecOp> &ops, uint64_t &flops) {
    std::vector<ExecStep> steps;
    for (const ExecOp &op : ops) {
      if (op.kind == ExecOp::Kind::Matmul || op.kind == ExecOp::Kind::GemvChain) {
        // A GEMV chain's jobs join the matmul segment in list order.
        std::vector<MatmulOp> one{op.matmul};
        const std::vector<MatmulOp> &list = op.kind == ExecOp::Kind::Matmul ? one : op.jobs;
        if (op.kind == ExecOp::Kind::GemvChain)
          check_gemv_chain(*this, op.jobs);
        // A chain is a step of its own; later matmuls start a new one.
        if (steps.empty() || !steps.back().matmul || steps.back().chain ||
            op.kind == ExecOp::Kind::GemvChain) {
          steps.emplace_back();
          steps.back().matmul = true;
          steps.back().chain = op.kind == ExecOp::Kind::GemvChain;
        }
        for (const MatmulOp &m : list) {
          validate_op(m);
          steps.back().ops.push_back(m);
          steps.back().res.push_back(ResolvedMatmul::from_op(m));
        }
      } else {
        steps.emplace_back();
        steps.back().elems = plan_exec_elem(*this, op);
      }
    }
    flops = 0;
    for (ExecStep &st : steps) {
      if (!st.matmul)
        continue;
      for (size_t i = 0; i < st.ops.size(); ++i)
        st.plans.push_back(plan_op(st.ops[i], st.res[i], false));
      if (!st.chain || !mark_chain(st.res, st.plans)) {
        mark_fusions(st.ops, st.res, st.plans);
        mark_groups(st.ops, st.res, st.plans);
      }
      for (size_t i = 0; i < st.ops.size(); ++i) {
        check_supported(KERNEL_SPECS[st.plans[i].kernel], st.res[i]);
        if (st.plans[i].role != 3 && st.plans[i].role != 4 && st.plans[i].role < 5)
          check_fusions(KERNEL_SPECS[st.plans[i].kernel], st.ops[i], st.res[i]);
      }
      flops += total_flops(st.res);
    }
    return steps;
  }
  ScratchNeed exec_need(const std::vector<ExecStep> &steps) const {
    ScratchNeed need;
    for (const ExecStep &st : steps)
      if (st.matmul)
        need.merge(total_need(st.res, st.plans));
    return need;
  }
  static bool exec_has_mlp(const std::vector<ExecStep> &steps) {
    for (const ExecStep &st : steps)
      if (st.matmul && has_mlp(st.plans))
        return true;
    return false;
  }
  void record_exec(const std::vector<ExecStep> &steps, Scratch &scratch, uint32_t *status,
                   hipStream_t stream) const {
    for (const ExecStep &st : steps) {
      if (st.matmul)
        record(st.ops, st.res, st.plans, scratch, status, stream);
      else
        record_elem(st.elems, stream);
    }
  }
  RunStats run_exec_impl(const std::vector<ExecOp> &ops) {
    if (ops.empty())
      fail("run_exec_ops: empty op list");
    ctx->make_current();
    uint64_t flops = 0;
    const std::vector<ExecStep> steps = plan_exec(ops, flops);
    Lease lease(this);
    Slot *slot = lease.s;
    const ScratchNeed need = exec_need(steps);
    slot->scratch.ensure(need.splitk, need.partial, need.counters);
    slot->scratch.ensure_mlp(need.mlp);
    slot->scratch.ensure_shadow(need.shadow);
    slot->scratch.ensure_barrier(need.barrier);
    hip_check(hipEventRecord(slot->start, slot->stream), "hipEventRecord");
    record_exec(steps, slot->scratch, slot->host_status, slot->stream);
    hip_check(hipEventRecord(slot->end, slot->stream), "hipEventRecord");
    hip_check(hipEventSynchronize(slot->end), "hipEventSynchronize");
    float ms = 0.f;
    hip_check(hipEventElapsedTime(&ms, slot->start, slot->end), "hipEventElapsedTime");
    if (exec_has_mlp(steps))
      check_host_status(slot->host_status, slot->scratch.mlp, slot->scratch.mlp_bytes);
    return RunStats{(uint64_t)((double)ms * 1e6), ops.size(), flops};
  }
  std::unique_ptr<PreparedOps> prepare_exec_impl(const Executor *owner,
                                                 const std::vector<ExecOp> &ops) {
    if (ops.empty())
      fail("prepare_exec_ops: empty op list");
    ctx->make_current();
    uint64_t flops = 0;
    auto steps = std::make_shared<std::vector<ExecStep>>(plan_exec(ops, flops));
    return capture(owner, ops.size(), flops, exec_need(*steps), exec_has_mlp(*steps),
                   [this, steps](Scratch &scratch, uint32_t *status, hipStream_t stream) {
                     record_exec(*steps, scratch, status, stream);
                   });
  }

  // ---- tuning (src/executor/tuning.rs) ----
  void load_store() {
    header = tune_header_line(*ctx);
    const std::string path = tune_store_path(*ctx);
    if (path.empty())
      return;
    std::ifstream in(path);
    if (!in)
      return;
    std::stringstream ss;
    ss << in.rdbuf();
    tuned = parse_tune_store(ss.str(), header);
  }

  void record_tuned(const TuneKey &key, const TuneEntry &e) {
    std::string text;
    {
      std::lock_guard<std::mutex> lock(tuned_mu);
      tuned[key] = e;
      text = format_tune_store(tuned, header);
    }
    const std::string path = tune_store_path(*ctx);
    if (path.empty())
      return;
    // Atomic rewrite: temp file + rename (pipeline/tuning.rs:157-199).
    const size_t slash = path.rfind('/');
    std::string dir = path.substr(0, slash);
    std::string parent = dir.substr(0, dir.rfind('/'));
    mkdir(parent.c_str(), 0755);
    mkdir(dir.c_str(), 0755);
    static std::atomic<uint64_t> next{0};
    const std::string tmp = path + ".tmp." + std::to_string(getpid()) + "." +
                            std::to_string(next.fetch_add(1));
    {
      std::ofstream out(tmp, std::ios::trunc);
      out << text;
      if (!out)
        return;
    }
    if (std::rename(tmp.c_str(), path.c_str()) != 0)
      std::remove(tmp.c_str());
  }

  bool is_tuned(const TuneKey &key) const {
    if (!selection.is_auto())
      return true;
    std::lock_guard<std::mutex> lock(tuned_mu);
    return tuned.count(key) != 0;
  }

  std::optional<uint64_t> run_forced_once(const MatmulOp &op, const ResolvedMatmul &d,
                                          size_t kernel, std::optional<uint32_t> splits) const {
    ExecutorImpl *self = const_cast<ExecutorImpl *>(this);
    Lease lease(self);
    OpPlan p;
    p.kernel = kernel;
    p.splitk2 = splits;
    return submit_and_wait(lease.s, {op}, {d}, {p});
  }

  void tune_op(const MatmulOp &op, const ResolvedMatmul &d) {
    std::vector<size_t> cands = tune_candidate_indices(d);
    if (cands.empty())
      fail("no tunable kernel fits this shape");
    const size_t heur =
        heuristic_kernel_index(ctx->cu_count(), d.batch, d.m, d.n, d.k, d.b_f16, d.packed_b);
    const double est_ms = (double)d.total_flops / 50e12 * 1e3;
    const uint32_t rounds = est_ms > 8.0 ? 2 : 4;
    (void)run_forced_once(op, d, std::count(cands.begin(), cands.end(), heur) ? heur : cands[0],
                          std::nullopt);
    std::vector<std::vector<uint64_t>> samples(cands.size());
    for (uint32_t round = 0; round <= rounds; ++round)
      for (size_t off = 0; off < cands.size(); ++off) {
        const size_t ci = candidate_at(cands.size(), round, off);
        auto ns = run_forced_once(op, d, cands[ci], std::nullopt);
        if (round > 0 && ns)
          samples[ci].push_back(*ns);
      }
    std::optional<uint64_t> heur_ns;
    size_t win = cands[0];
    std::optional<uint64_t> win_ns;
    const bool log = std::getenv("TA_LOG") != nullptr;
    for (size_t i = 0; i < cands.size(); ++i) {
      auto md = median(samples[i]);
      if (log)
        std::fprintf(stderr, "tensor-ash: tune B=%u %ux%ux%u candidate %s: median %.2f us (%zu samples)%s\n",
                     d.batch, d.m, d.n, d.k, KERNEL_SPECS[cands[i]].name,
                     md ? (double)*md / 1e3 : -1.0, samples[i].size(),
                     cands[i] == heur ? " [heuristic]" : "");
      if (!md)
        continue;
      if (cands[i] == heur)
        heur_ns = md;
      if (!win_ns || *md < *win_ns) {
        win_ns = md;
        win = cands[i];
      }
    }
    if (!win_ns)
      fail("no candidate produced a measurement");
    if (heur_ns && (double)*win_ns >= (double)*heur_ns * 0.98) {
      win = heur;
      win_ns = heur_ns;
    }
    // Reduction pass: probe split-K against the DP winner on deep-K,
    // few-tile shapes (executor/tuning.rs:203-250).
    std::optional<uint32_t> best_splits;
    const KernelSpec &s1 = splitk_stage1_spec(d.m, d.n, d.k);
    const uint64_t tiles = (uint64_t)d.batch * div_ceil(d.m, s1.tile_m) * div_ceil(d.n, s1.tile_n);
    if (!d.b_f16 && !d.packed_b && d.k >= 1024 && tiles < ctx->cu_count()) {
      std::optional<uint64_t> best;
      for (uint32_t splits : {4u, 8u, 16u, 32u, 64u, 128u}) {
        if (d.k / splits < 128 || !auto_route_fits(d.batch, d.m, d.n, d.k, splits))
          continue;
        std::vector<uint64_t> ss;
        for (uint32_t r = 0; r <= rounds; ++r) {
          auto ns = run_forced_once(op, d, registry_index(s1.name), splits);
          if (r > 0 && ns)
            ss.push_back(*ns);
        }
        auto md = median(ss);
        if (log)
          std::fprintf(stderr, "tensor-ash: tune B=%u %ux%ux%u split-K %s x %u: median %.2f us\n",
                       d.batch, d.m, d.n, d.k, s1.name, splits, md ? (double)*md / 1e3 : -1.0);
        if (md && (!best || *md < *best)) {
          best = md;
          best_splits = splits;
        }
      }
      if (!best || (double)*best >= (double)*win_ns * 0.98)
        best_splits.reset();
    }
    record_tuned(TuneKey{d.batch, d.m, d.n, d.k, d.b_f16}, TuneEntry{win, best_splits});
    if (std::getenv("TA_LOG"))
      std::fprintf(stderr, "tensor-ash: tuned B=%u %ux%ux%u: %s%s\n", d.batch, d.m, d.n, d.k,
                   KERNEL_SPECS[win].name,
                   best_splits ? (" + splitk2=" + std::to_string(*best_splits)).c_str() : "");
  }

  // ---- run_ops (src/executor/dispatch.rs:87-188) ----
  RunStats run_ops_impl(const std::vector<MatmulOp> &ops, bool graph) {
    if (ops.empty())
      return RunStats{std::nullopt, 0, 0};
    if (ops.size() > config.max_calls_per_submit)
      fail("run_ops: " + std::to_string(ops.size()) + " ops > max_calls_per_submit " +
           std::to_string(config.max_calls_per_submit));
    ctx->make_current();
    for (const auto &op : ops)
      validate_op(op);
    std::vector<ResolvedMatmul> res;
    res.reserve(ops.size());
    for (const auto &op : ops)
      res.push_back(ResolvedMatmul::from_op(op));
    const uint64_t flops = total_flops(res);

    if (config.tune && ops.size() == 1 && !ops[0].call.accumulate && ops[0].epilogue.is_none() &&
        !ops[0].has_decode_fusion() && !res[0].a_f16 && !res[0].packed_b) {
      const ResolvedMatmul &d = res[0];
      const TuneKey key{d.batch, d.m, d.n, d.k, d.b_f16};
      if (!is_tuned(key)) {
        try {
          tune_op(ops[0], d);
        } catch (const Error &e) {
          std::fprintf(stderr, "tensor-ash: tuning failed for B=%u %ux%ux%u: %s\n", d.batch,
                       d.m, d.n, d.k, e.what());
        }
      }
    }

    // Split-K eligibility.  The reference offers it to plain ops only
    // (src/executor/mod.rs:125-139) and also excludes multi-op run_ops
    // submissions, whose ops share one scratch with no barriers between
    // them.  Here each stream lane has its own scratch and runs in stream
    // order, and the reduce applies the fused epilogue (accumulate, bias,
    // activation, binary with D) once to the finished plane sum, so every
    // f32 op may take the split-K route: a deep-K skinny GEMM with an
    // epilogue would otherwise run a handful of workgroups on 256 CUs.
    std::vector<OpPlan> plans;
    for (size_t i = 0; i < ops.size(); ++i)
      plans.push_back(plan_op(ops[i], res[i], true));
    if (graph)
      mark_fusions(ops, res, plans);
    if (!graph && plans.size() == 1 && plans[0].splitk2)
      return run_split_k2(ops[0], *plans[0].splitk2, "run_ops", true);
    const uint32_t lanes = graph ? 1u : run_ops_lanes(res, plans);
    if (lanes == 1)
      mark_groups(ops, res, plans);

    Lease lease(this);
    const uint64_t ns = lanes > 1 ? submit_concurrent(lease.s, ops, res, plans)
                                  : submit_and_wait(lease.s, ops, res, plans);
    return RunStats{ns, ops.size(), flops};
  }

  // Lanes for a run_ops submission of independent ops.  Forking onto side
  // streams and joining back costs ~40 us on this platform (measured with
  // four 28 us kernels: 114 us serial, 71 us over four streams), and an op
  // whose grid covers the CUs (split-K, decode GEMV and large-tile routes
  // are planned that way) gains nothing from company.  So the ops are
  // spread only when those whose grids leave most CUs idle would, run
  // back to back, take well over that beyond the longest of them; an op's
  // time is estimated from flops and bytes at sustained rates, scaled by
  // the share of the CUs its grid occupies.  TA_RUN_OPS_LANES fixes the
  // lane count (1 = serial; route control).
  uint32_t run_ops_lanes(const std::vector<ResolvedMatmul> &res,
                         const std::vector<OpPlan> &plans) const {
    if (res.size() < 2)
      return 1;
    if (const char *env = std::getenv("TA_RUN_OPS_LANES"))
      return (uint32_t)std::clamp<unsigned long>(std::strtoul(env, nullptr, 10), 1, kRunOpsLanes);
    const double cus = ctx->cu_count();
    double total = 0.0, longest = 0.0;
    size_t small = 0;
    for (size_t i = 0; i < res.size(); ++i) {
      const ResolvedMatmul &d = res[i];
      const KernelSpec &s = KERNEL_SPECS[plans[i].kernel];
      if (plans[i].splitk2 || s.is_gemv())
        continue;
      const double tiles = (double)d.batch * div_ceil(d.m, s.tile_m) * div_ceil(d.n, s.tile_n);
      if (tiles >= cus / 2)
        continue;
      const double bytes = (d.a_f16 ? 2.0 : 4.0) * d.batch * d.m * d.k +
                           (d.b_f16 ? 2.0 : 4.0) * (d.batch_stride_b ? d.batch : 1) * d.k * d.n +
                           4.0 * d.batch * d.m * d.n;
      const double rate = d.b_f16 ? 300e12 : 80e12; // sustained flop/s on the whole chip
      const double us =
          std::max((double)d.total_flops / rate, bytes / 4e12) * 1e6 * cus / tiles + 5.0;
      total += us;
      longest = std::max(longest, us);
      ++small;
    }
    return small >= 2 && total - longest > 60.0 ? (uint32_t)std::min(kRunOpsLanes, res.size())
                                                : 1u;
  }

  // ---- split-K (src/executor/reduction.rs:21-70) ----
  // Validates the op and resolves the split count (0 = default).  `fn`
  // names the entry point in error texts; the call form keeps the
  // reference's refusal of accumulate, the op form applies it in the
  // reduce with the rest of the epilogue.
  uint32_t split_k2_splits(const MatmulOp &op, uint32_t num_k_splits, ResolvedMatmul &d,
                           const std::string &fn, bool allow_accumulate) const {
    validate_op(op);
    if (op.call.accumulate && !allow_accumulate)
      fail(fn + ": accumulate=true is not supported");
    if (op.has_decode_fusion())
      fail(fn + ": decode fusions (normed A, RoPE/scatter store) need a decode GEMV route");
    d = ResolvedMatmul::from_op(op);
    if (num_k_splits > 0xFFFF)
      fail(fn + ": num_k_splits=" + std::to_string(num_k_splits) + " out of range [1, 65535]");
    if (num_k_splits > d.k)
      fail(fn + ": num_k_splits=" + std::to_string(num_k_splits) + " exceeds K=" +
           std::to_string(d.k));
    if (d.a_f16 || d.b_f16)
      fail(fn + ": split-K stage 1 reads f32 A and B only");
    const uint32_t splits =
        num_k_splits == 0 ? default_num_k_splits(ctx->cu_count(), d.batch, d.m, d.n, d.k)
                          : num_k_splits;
    if (splits > 1) {
      validate_scratch_geometry(d.batch, d.m, d.n, d.k, splits);
      if ((uint64_t)d.batch * splits > 65535)
        fail("split-K2 dispatch grid Z (" + std::to_string((uint64_t)d.batch * splits) +
             ") exceeds 65535");
    }
    return splits;
  }

  // The route of an explicit split count: the split-K stage-1 tile plus
  // the reduce for splits > 1, else the data-parallel route (the same
  // plan run_ops gives an op that may not split), which needs no scratch
  // for f32 operands.  The allocating and the allocation-free entry
  // points share it, so they launch the same kernels.
  OpPlan split_k2_plan(const MatmulOp &op, const ResolvedMatmul &d, uint32_t splits) const {
    if (splits <= 1)
      return plan_op(op, d, false);
    OpPlan p;
    p.kernel = registry_index(splitk_stage1_spec(d.m, d.n, d.k).name);
    p.splitk2 = splits;
    return p;
  }

  RunStats run_split_k2(const MatmulOp &op, uint32_t num_k_splits, const std::string &fn,
                        bool allow_accumulate) {
    ctx->make_current();
    ResolvedMatmul d;
    const uint32_t splits = split_k2_splits(op, num_k_splits, d, fn, allow_accumulate);
    const OpPlan p = split_k2_plan(op, d, splits);
    Lease lease(this);
    const uint64_t ns = submit_and_wait(lease.s, {op}, {d}, {p});
    return RunStats{ns, 1, d.total_flops};
  }

  // The same launches with the partial planes in the device's fixed
  // scratch array instead of slot memory: nothing is allocated, on the
  // device or pinned.  Calls on one device are serialised here, from the
  // first launch until the stream has drained, because they share the
  // array; the planes need no clearing (every element is stored before
  // the reduce reads it).
  RunStats run_split_k2_noalloc(const MatmulCall &call, uint32_t num_k_splits) {
    ctx->make_current();
    const std::string fn = "run_matmuls_split_k2_noalloc";
    const MatmulOp op(call);
    ResolvedMatmul d;
    const uint32_t splits = split_k2_splits(op, num_k_splits, d, fn, false);
    const OpPlan p = split_k2_plan(op, d, splits);
    const ScratchNeed need = scratch_need(d, p);
    if (need.partial || need.counters)
      fail("internal: " + fn + " route needs slot scratch");
    if (need.splitk > TA_FIXED_SCRATCH_BYTES)
      fail(fn + ": partial planes need " + std::to_string(need.splitk) + " bytes (B=" +
           std::to_string(d.batch) + " " + std::to_string(d.m) + "x" + std::to_string(d.n) +
           ", " + std::to_string(splits) + " splits) > the fixed scratch of " +
           std::to_string(TA_FIXED_SCRATCH_BYTES) + " bytes");
    void *base = nullptr;
    hip_check(fixed_scratch_address(ctx->device(), &base), "hipGetSymbolAddress (fixed scratch)");
    Scratch fixed;
    fixed.splitk = base;
    fixed.splitk_bytes = TA_FIXED_SCRATCH_BYTES;
    std::lock_guard<std::mutex> serial(fixed_scratch_mutex(ctx->device()));
    Lease lease(this);
    const uint64_t ns = submit_on(lease.s, {op}, {d}, {p}, fixed);
    return RunStats{ns, 1, d.total_flops};
  }

  // ---- prepared (src/executor/prepared.rs:67-160) ----
  std::unique_ptr<PreparedOps> prepare_impl(const Executor *owner,
                                            const std::vector<MatmulOp> &ops, bool graph) {
    if (ops.empty())
      fail("prepare_ops: empty op batch");
    if (ops.size() > config.max_calls_per_submit)
      fail("prepare_ops: " + std::to_string(ops.size()) + " ops > max_calls_per_submit " +
           std::to_string(config.max_calls_per_submit));
    ctx->make_current();
    for (const auto &op : ops)
      validate_op(op);
    std::vector<ResolvedMatmul> res;
    for (const auto &op : ops)
      res.push_back(ResolvedMatmul::from_op(op));
    const uint64_t flops = total_flops(res);
    // Data-parallel routes only, like the reference: split-K would need
    // its scratch baked into the graph for the handle's lifetime.
    std::vector<OpPlan> plans;
    for (size_t i = 0; i < res.size(); ++i)
      plans.push_back(plan_op(ops[i], res[i], false));
    if (graph)
      mark_fusions(ops, res, plans);
    mark_groups(ops, res, plans);
    for (size_t i = 0; i < ops.size(); ++i)
      check_supported(KERNEL_SPECS[plans[i].kernel], res[i]);

    return capture(owner, ops.size(), flops, total_need(res, plans), has_mlp(plans),
                   [&](Scratch &scratch, uint32_t *status, hipStream_t stream) {
                     record(ops, res, plans, scratch, status, stream);
                   });
  }

  // Record once into a hipGraph on a private stream, with graph-owned
  // scratch zeroed outside the capture (no memset nodes).
  std::unique_ptr<PreparedOps>
  capture(const Executor *owner, size_t n_calls, uint64_t flops, const ScratchNeed &need,
          bool mlp, const std::function<void(Scratch &, uint32_t *, hipStream_t)> &rec) {
    std::unique_ptr<PreparedOps> p(new PreparedOps());
    p->exec_ = owner;
    p->n_calls_ = n_calls;
    p->flops_ = flops;
    hipStream_t stream = nullptr;
    hip_check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
    p->stream_ = stream;
    hipEvent_t e0, e1;
    hip_check(hipEventCreate(&e0), "hipEventCreate");
    p->ev_start_ = e0;
    hip_check(hipEventCreate(&e1), "hipEventCreate");
    p->ev_end_ = e1;
    Scratch scratch;
    scratch.ensure(need.splitk, need.partial, need.counters);
    scratch.ensure_mlp(need.mlp);
    scratch.ensure_shadow(need.shadow);
    scratch.ensure_barrier(need.barrier);
    p->scratch_ = {scratch.splitk, scratch.partial, scratch.counters, scratch.mlp, scratch.shadow,
                   scratch.barrier};
    p->mlp_scratch_ = scratch.mlp;
    p->mlp_bytes_ = scratch.mlp_bytes;
    if (mlp)
      p->status_ = alloc_host_status();

    hipGraph_t g = nullptr;
    hip_check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal),
              "hipStreamBeginCapture");
    try {
      rec(scratch, static_cast<uint32_t *>(p->status_), stream);
    } catch (...) {
      (void)hipStreamEndCapture(stream, &g);
      if (g)
        (void)hipGraphDestroy(g);
      throw;
    }
    hip_check(hipStreamEndCapture(stream, &g), "hipStreamEndCapture");
    hipGraphExec_t ge = nullptr;
    hipError_t err = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    hip_check(err, "hipGraphInstantiate");
    p->graph_exec_ = ge;
    return p;
  }

  // ---- transfers (src/executor/transfer.rs) ----
  void copy_to_device(const void *src, uint64_t bytes, const Tensor &dst, const char *op) {
    if (bytes > dst.size_bytes())
      fail(std::string(op) + ": " + std::to_string(bytes) + " bytes > tensor capacity " +
           std::to_string(dst.size_bytes()));
    Lease lease(this);
    hip_check(hipMemcpyAsync(dst.device_ptr(), src, bytes, hipMemcpyHostToDevice, lease.s->stream),
              "hipMemcpyAsync (upload)");
    hip_check(hipStreamSynchronize(lease.s->stream), "hipStreamSynchronize");
  }
};

// ---------------------------------------------------------------- Executor

Executor::Executor(std::shared_ptr<Context> ctx, KernelSelection selection, ExecutorConfig config)
    : impl_(new ExecutorImpl()) {
  impl_->ctx = std::move(ctx);
  impl_->selection = selection;
  config.n_slots = std::max<size_t>(1, config.n_slots);
  config.max_calls_per_submit = std::max<uint32_t>(1, config.max_calls_per_submit);
  impl_->config = config;
  impl_->ctx->make_current();
  for (size_t i = 0; i < config.n_slots; ++i) {
    Slot *s = new Slot();
    hip_check(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking), "hipStreamCreate");
    hip_check(hipEventCreate(&s->start), "hipEventCreate");
    hip_check(hipEventCreate(&s->end), "hipEventCreate");
    s->host_status = alloc_host_status();
    impl_->all_slots.push_back(s);
    impl_->free_slots.push_back(s);
  }
  impl_->load_store();
}

namespace {
bool env_tune() {
  const char *v = std::getenv("ML_TUNE");
  if (!v)
    return false;
  std::string s = v;
  for (auto &c : s)
    c = (char)std::tolower((unsigned char)c);
  return s == "1" || s == "on" || s == "true";
}
} // namespace

Executor::Executor(std::shared_ptr<Context> ctx, KernelSelection selection, size_t n_slots,
                   uint32_t max_calls_per_submit)
    : Executor(std::move(ctx), selection, ExecutorConfig{n_slots, max_calls_per_submit, env_tune()}) {}

Executor::~Executor() {
  if (!impl_)
    return;
  (void)hipSetDevice(impl_->ctx->device());
  for (Slot *s : impl_->all_slots) {
    (void)hipStreamSynchronize(s->stream);
    for (SideLane &l : s->side) {
      (void)hipStreamSynchronize(l.stream);
      l.scratch.release();
      (void)hipEventDestroy(l.done);
      (void)hipStreamDestroy(l.stream);
    }
    if (s->fork)
      (void)hipEventDestroy(s->fork);
    s->scratch.release();
    (void)hipEventDestroy(s->start);
    (void)hipEventDestroy(s->end);
    (void)hipStreamDestroy(s->stream);
    if (s->host_status)
      (void)hipHostFree(s->host_status);
    delete s;
  }
}

const std::shared_ptr<Context> &Executor::context() const { return impl_->ctx; }

RunStats Executor::run_matmuls(const std::vector<MatmulCall> &calls) const {
  std::vector<MatmulOp> ops;
  for (const auto &c : calls)
    ops.emplace_back(c);
  return impl_->run_ops_impl(ops, false);
}
RunStats Executor::run_matmul_graph(const std::vector<MatmulCall> &calls) const {
  std::vector<MatmulOp> ops;
  for (const auto &c : calls)
    ops.emplace_back(c);
  return impl_->run_ops_impl(ops, true);
}
RunStats Executor::run_ops(const std::vector<MatmulOp> &ops) const {
  return impl_->run_ops_impl(ops, false);
}
RunStats Executor::run_op_graph(const std::vector<MatmulOp> &ops) const {
  return impl_->run_ops_impl(ops, true);
}
RunStats Executor::run_gemv_chain(const std::vector<MatmulOp> &jobs) const {
  check_gemv_chain(*impl_, jobs);
  return impl_->run_chain_impl(jobs);
}

RunStats Executor::run_matmuls_split_k2(const MatmulCall &call, uint32_t num_k_splits) const {
  return impl_->run_split_k2(MatmulOp(call), num_k_splits, "run_matmuls_split_k2", false);
}

RunStats Executor::run_op_split_k2(const MatmulOp &op, uint32_t num_k_splits) const {
  return impl_->run_split_k2(op, num_k_splits, "run_op_split_k2", true);
}

RunStats Executor::run_matmuls_split_k2_noalloc(const MatmulCall &call,
                                                uint32_t num_k_splits) const {
  return impl_->run_split_k2_noalloc(call, num_k_splits);
}

// ---- model ops (src/executor/elementwise/ops.rs) ----
namespace {
void ensure_f32(const Tensor &t, const std::string &op, const char *role) {
  if (t.dtype() != DType::F32)
    fail(op + ": " + role + " must be f32 storage (got " + dtype_name(t.dtype()) + ")");
}
void ensure_same_shape(const std::string &op, const Tensor &in, const Tensor &out) {
  if (in.shape() != out.shape())
    fail(op + ": output shape " + fmt_shape(out.shape()) + " must equal input shape " +
         fmt_shape(in.shape()));
}
// elementwise/mod.rs:391-398.
std::pair<uint32_t, uint32_t> rows_cols(const Tensor &t, const std::string &op) {
  const uint32_t cols = t.shape().back();
  const uint64_t rows = t.len() / cols;
  if (rows > UINT32_MAX)
    fail(op + ": row count " + std::to_string(rows) + " exceeds u32");
  return {(uint32_t)rows, cols};
}
bool io_f16(const std::string &op, const Tensor &in, const Tensor &out) {
  if (in.dtype() != out.dtype())
    fail(op + ": input (" + dtype_name(in.dtype()) + ") and output (" + dtype_name(out.dtype()) +
         ") must share a storage type");
  return in.dtype() == DType::F16;
}
uint32_t grid_for(uint64_t items, uint32_t per_group, uint32_t cus) {
  return (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>((items + per_group - 1) / per_group,
                                                            64ull * cus));
}
template <class T> ElemLaunch elem(const char *symbol, uint32_t groups, const T &args) {
  ElemLaunch l;
  l.symbol = symbol;
  l.groups = groups;
  l.args.resize(sizeof(T));
  std::memcpy(l.args.data(), &args, sizeof(T));
  return l;
}

ElemLaunch plan_softmax(ExecutorImpl &e, const Tensor &input, const Tensor &output, float scale,
                        SoftmaxMask mask) {
  const std::string op = "run_softmax_rows";
  e.validate_tensor(&input, "input");
  e.validate_tensor(&output, "output");
  ensure_f32(input, op, "input");
  ensure_f32(output, op, "output");
  ensure_same_shape(op, input, output);
  auto [rows, cols] = rows_cols(input, op);
  SoftmaxArgs a{};
  a.in = static_cast<const float *>(input.device_ptr());
  a.out = static_cast<float *>(output.device_ptr());
  a.rows = rows;
  a.cols = cols;
  a.scale = scale;
  a.rows_per_group = 1;
  switch (mask.kind) {
  case SoftmaxMask::Kind::Full:
    a.valid_base = cols;
    break;
  case SoftmaxMask::Kind::Prefix:
    a.valid_base = std::min(mask.valid, cols);
    break;
  case SoftmaxMask::Kind::Causal:
    if (mask.rows_per_group == 0 || rows % mask.rows_per_group != 0)
      fail(op + ": rows_per_group " + std::to_string(mask.rows_per_group) +
           " must divide rows " + std::to_string(rows));
    a.valid_base = mask.prefix;
    a.rows_per_group = mask.rows_per_group;
    a.causal = 1;
    break;
  }
  return elem("ta_softmax_rows", grid_for(rows, 1, e.ctx->cu_count()), a);
}

ElemLaunch plan_norm(ExecutorImpl &e, const std::string &op, const Tensor &input,
                     const Tensor &weight, const Tensor *bias, const Tensor &output, float eps) {
  e.validate_tensor(&input, "input");
  e.validate_tensor(&output, "output");
  e.validate_tensor(&weight, "weight");
  const bool f16 = io_f16(op, input, output);
  ensure_f32(weight, op, "weight");
  if (bias) {
    e.validate_tensor(bias, "bias");
    ensure_f32(*bias, op, "bias");
    if (f16)
      fail(op + ": f16 activations are supported for RMSNorm only (no f16 LayerNorm kernel)");
  }
  ensure_same_shape(op, input, output);
  auto [rows, cols] = rows_cols(input, op);
  if (weight.len() != cols)
    fail(op + ": weight length " + std::to_string(weight.len()) + " != row length " +
         std::to_string(cols));
  if (bias && bias->len() != cols)
    fail(op + ": bias length " + std::to_string(bias->len()) + " != row length " +
         std::to_string(cols));
  NormArgs a{};
  a.in = input.device_ptr();
  a.out = output.device_ptr();
  a.weight = static_cast<const float *>(weight.device_ptr());
  a.bias = bias ? static_cast<const float *>(bias->device_ptr()) : nullptr;
  a.rows = rows;
  a.cols = cols;
  a.eps = eps;
  a.io_f16 = f16 ? 1u : 0u;
  return elem("ta_norm_rows", grid_for(rows, 1, e.ctx->cu_count()), a);
}

// ops.rs:177-207 (rope_tokens): the token count of `input` under desc,
// with rot_dim and table coverage checked.
uint64_t rope_tokens(const std::string &op, const Tensor &input, const Tensor &table,
                     const RopeDesc &desc) {
  if (desc.rot_dim < 2 || desc.rot_dim % 2 != 0 || desc.rot_dim > desc.head_dim)
    fail(op + ": rot_dim " + std::to_string(desc.rot_dim) +
         " must be even, >= 2, and <= head_dim " + std::to_string(desc.head_dim));
  const uint64_t vec_elems = (uint64_t)desc.heads * desc.head_dim;
  if (vec_elems == 0 || input.len() % vec_elems != 0)
    fail(op + ": input length " + std::to_string(input.len()) +
         " is not a multiple of heads*head_dim " + std::to_string(vec_elems));
  const uint64_t tokens = input.len() / vec_elems;
  if (tokens > UINT32_MAX)
    fail(op + ": token count exceeds u32");
  const uint64_t needed = ((uint64_t)desc.pos_base + tokens) * desc.rot_dim;
  if (table.len() < needed)
    fail(op + ": table length " + std::to_string(table.len()) + " < required " +
         std::to_string(needed) + " (pos_base " + std::to_string(desc.pos_base) + " + " +
         std::to_string(tokens) + " tokens, rot_dim " + std::to_string(desc.rot_dim) + ")");
  return tokens;
}

ElemLaunch plan_rope(ExecutorImpl &e, const Tensor &input, const Tensor &table,
                     const Tensor &output, const RopeDesc &desc) {
  const std::string op = "run_rope";
  e.validate_tensor(&input, "input");
  e.validate_tensor(&output, "output");
  e.validate_tensor(&table, "table");
  const bool f16 = io_f16(op, input, output);
  ensure_f32(table, op, "table");
  ensure_same_shape(op, input, output);
  const uint64_t tokens = rope_tokens(op, input, table, desc);
  RopeArgs a{};
  a.in = input.device_ptr();
  a.out = output.device_ptr();
  a.table = static_cast<const float *>(table.device_ptr());
  a.pos_addr = reinterpret_cast<const uint32_t *>(desc.pos_addr);
  a.tokens = (uint32_t)tokens;
  a.heads = desc.heads;
  a.head_dim = desc.head_dim;
  a.rot_dim = desc.rot_dim;
  a.pos_base = desc.pos_base;
  a.io_f16 = f16 ? 1u : 0u;
  a.table_len = table.len();
  const uint64_t pairs = tokens * desc.heads * (desc.rot_dim / 2);
  return elem("ta_rope", grid_for(pairs, 256, e.ctx->cu_count()), a);
}

ElemLaunch plan_copy(ExecutorImpl &e, const Tensor &src, const Tensor &dst, const CopyDesc &desc) {
  const std::string op = "run_copy_strided";
  e.validate_tensor(&src, "src");
  e.validate_tensor(&dst, "dst");
  // ops.rs:387-437.
  if (src.buffer_id() == dst.buffer_id())
    fail(op + ": src and dst must be different tensors");
  for (uint32_t x : desc.extent)
    if (x == 0)
      fail(op + ": extent [" + std::to_string(desc.extent[0]) + ", " +
           std::to_string(desc.extent[1]) + ", " + std::to_string(desc.extent[2]) +
           "] has a zero axis");
  auto max_index = [&](uint32_t offset, const std::array<uint32_t, 3> &strides) {
    uint64_t m = offset;
    for (int i = 0; i < 3; ++i)
      m += (uint64_t)(desc.extent[i] - 1) * strides[i];
    return m;
  };
  if (max_index(desc.src_offset, desc.src_strides) >= src.len())
    fail(op + ": source access reaches element " +
         std::to_string(max_index(desc.src_offset, desc.src_strides)) + " but src has " +
         std::to_string(src.len()));
  if (max_index(desc.dst_offset, desc.dst_strides) >= dst.len())
    fail(op + ": destination access reaches element " +
         std::to_string(max_index(desc.dst_offset, desc.dst_strides)) + " but dst has " +
         std::to_string(dst.len()));
  const uint64_t total = (uint64_t)desc.extent[0] * desc.extent[1] * desc.extent[2];
  if (total > UINT32_MAX)
    fail(op + ": extent product exceeds u32");
  CopyArgs a{};
  a.src = src.device_ptr();
  a.dst = dst.device_ptr();
  a.pos_addr = reinterpret_cast<const uint32_t *>(desc.pos_addr);
  for (int i = 0; i < 3; ++i) {
    a.extent[i] = desc.extent[i];
    a.src_strides[i] = desc.src_strides[i];
    a.dst_strides[i] = desc.dst_strides[i];
  }
  a.src_offset = desc.src_offset;
  a.dst_offset = desc.dst_offset;
  a.pos_scale = desc.pos_scale;
  a.src_f16 = src.dtype() == DType::F16 ? 1u : 0u;
  a.dst_f16 = dst.dtype() == DType::F16 ? 1u : 0u;
  a.dst_len = dst.len();
  return elem("ta_copy_strided", grid_for(total, 256, e.ctx->cu_count()), a);
}

// flash.rs:66-250 (plan_flash_attention): the same checks in the same
// order, then the head-dimension / storage variant.
ElemLaunch plan_flash(ExecutorImpl &e, const Tensor &q, const Tensor &kt, const Tensor &v,
                      const Tensor &out, const FlashAttentionDesc &desc) {
  const std::string op = "run_flash_attention";
  e.validate_tensor(&q, "q");
  e.validate_tensor(&out, "out");
  const bool io16 = io_f16(op, q, out);
  e.validate_tensor(&kt, "kt");
  e.validate_tensor(&v, "v");
  if (kt.dtype() != v.dtype())
    fail(op + ": kt (" + dtype_name(kt.dtype()) + ") and v (" + dtype_name(v.dtype()) +
         ") must share a storage type");
  const bool kv16 = kt.dtype() == DType::F16;
  if (kt.shape().size() != 3)
    fail(op + ": kt must be [H_kv, dh, T_max], got " + fmt_shape(kt.shape()));
  if (v.shape().size() != 3)
    fail(op + ": v must be [H_kv, T_max, dh], got " + fmt_shape(v.shape()));
  const uint32_t kv_heads = kt.shape()[0], dh = kt.shape()[1], t_max = kt.shape()[2];
  if (v.shape()[1] != t_max || v.shape()[0] != kv_heads || v.shape()[2] != dh)
    fail(op + ": inconsistent cache shapes kt " + fmt_shape(kt.shape()) + ", v " +
         fmt_shape(v.shape()));
  uint32_t heads = 0, t_q = 0, q_hs = 0, q_rs = 0;
  if (desc.token_major_heads) {
    heads = *desc.token_major_heads;
    if (heads == 0)
      fail(op + ": token_major_heads must be nonzero");
    t_q = q.shape().empty() ? 0 : q.shape()[0];
    const uint64_t want = (uint64_t)t_q * heads * dh;
    if (t_q == 0 || q.len() != want)
      fail(op + ": token-major q " + fmt_shape(q.shape()) + " does not hold [T=" +
           std::to_string(t_q) + ", H=" + std::to_string(heads) + ", dh=" + std::to_string(dh) +
           "]");
    q_hs = dh;
    q_rs = heads * dh;
  } else {
    if (q.shape().size() != 3)
      fail(op + ": q must be [H, T_q, dh], got " + fmt_shape(q.shape()));
    heads = q.shape()[0];
    t_q = q.shape()[1];
    if (q.shape()[2] != dh)
      fail(op + ": q dh " + std::to_string(q.shape()[2]) + " != cache dh " + std::to_string(dh) +
           " (q " + fmt_shape(q.shape()) + ", kt " + fmt_shape(kt.shape()) + ")");
    q_hs = t_q * dh;
    q_rs = dh;
  }
  uint32_t o_hs = q_hs, o_rs = q_rs;
  if (desc.out_token_major_heads) {
    const uint32_t oh = *desc.out_token_major_heads;
    if (oh == 0)
      fail(op + ": out_token_major_heads must be nonzero");
    if (oh != heads)
      fail(op + ": out_token_major_heads " + std::to_string(oh) + " != q heads " +
           std::to_string(heads));
    if (out.len() != (uint64_t)t_q * oh * dh)
      fail(op + ": token-major out " + fmt_shape(out.shape()) + " does not hold [T=" +
           std::to_string(t_q) + ", H=" + std::to_string(oh) + ", dh=" + std::to_string(dh) +
           "]");
    o_hs = dh;
    o_rs = oh * dh;
  } else if (desc.token_major_heads) {
    if (out.len() != q.len())
      fail(op + ": out shape " + fmt_shape(out.shape()) + " must match token-major q " +
           fmt_shape(q.shape()));
  } else if (out.shape() != q.shape()) {
    fail(op + ": out shape " + fmt_shape(out.shape()) + " must equal q shape " +
         fmt_shape(q.shape()));
  }
  if (kv_heads == 0 || heads % kv_heads != 0)
    fail(op + ": H=" + std::to_string(heads) + " must be a multiple of H_kv=" +
         std::to_string(kv_heads));
  if (desc.kv_len > t_max)
    fail(op + ": kv_len " + std::to_string(desc.kv_len) + " exceeds cache T_max " +
         std::to_string(t_max));
  if (dh != 64 && dh != 128)
    fail(op + ": head dimension " + std::to_string(dh) +
         " unsupported (compiled variants: 64, 128)");
  if (io16 && !kv16)
    fail(op + ": f16 q/out are compiled for f16 KV caches only (kv " + dtype_name(kt.dtype()) +
         ", dh " + std::to_string(dh) + ")");
  FlashArgs a{};
  a.q = q.device_ptr();
  a.kt = kt.device_ptr();
  a.v = v.device_ptr();
  a.out = out.device_ptr();
  a.t_q = t_q;
  a.t_max = t_max;
  a.kv_len = desc.kv_len;
  a.pos_base = desc.pos_base;
  a.group_size = heads / kv_heads;
  a.scale = desc.scale;
  a.q_head_stride = q_hs;
  a.q_row_stride = q_rs;
  a.o_head_stride = o_hs;
  a.o_row_stride = o_rs;
  a.heads = heads;
  const uint32_t rows = ta_flash_rows((int)dh); // query rows per workgroup
  a.q_tiles = (t_q + rows - 1) / rows;
  const uint64_t groups = (uint64_t)a.q_tiles * heads;
  if (groups == 0 || groups > UINT32_MAX)
    fail(op + ": empty or oversized launch (T_q " + std::to_string(t_q) + ", H " +
         std::to_string(heads) + ")");
  const char *sym = io16 ? (dh == 64 ? "ta_flash_attention_io16_dh64"
                                     : "ta_flash_attention_io16_dh128")
                   : kv16 ? (dh == 64 ? "ta_flash_attention_kv16_dh64"
                                      : "ta_flash_attention_kv16_dh128")
                          : (dh == 64 ? "ta_flash_attention_dh64" : "ta_flash_attention_dh128");
  ElemLaunch l = elem(sym, (uint32_t)groups, a);
  l.threads = (uint32_t)ta_flash_threads((int)dh); // QB query blocks x KP key parts, 64 lanes each
  return l;
}

// ops.rs:467-500 (plan_argmax): f32 input, any shape, read flat.
ElemLaunch plan_argmax(ExecutorImpl &e, const Tensor &input, const U32Cell &result) {
  const std::string op = "run_argmax";
  e.validate_tensor(&input, "input");
  ensure_f32(input, op, "input");
  if (result.context() != e.ctx.get())
    fail(op + ": result buffer belongs to a different context");
  if (input.len() > UINT32_MAX)
    fail(op + ": input length exceeds u32");
  if (input.len() == 0)
    fail(op + ": input is empty");
  ArgmaxArgs a{};
  a.in = static_cast<const float *>(input.device_ptr());
  a.result = reinterpret_cast<uint32_t *>(result.device_address());
  a.n = (uint32_t)input.len();
  ElemLaunch l = elem("ta_argmax_f32", 1, a);
  l.threads = 1024;
  return l;
}

// ops.rs:529-595 (plan_embed_gather): table [vocab, embd] f32 or f16, out
// [embd] or [t, embd] f32 or f16, ids from the cell's first t slots.
ElemLaunch plan_embed_gather(ExecutorImpl &e, const U32Cell &tokens, const Tensor &table,
                             const Tensor &out) {
  const std::string op = "run_embed_gather";
  e.validate_tensor(&table, "table");
  e.validate_tensor(&out, "out");
  if (tokens.context() != e.ctx.get())
    fail(op + ": token buffer belongs to a different context");
  if (table.shape().size() != 2)
    fail(op + ": table must be [vocab, embd], got " + fmt_shape(table.shape()));
  const uint32_t vocab = table.shape()[0], embd = table.shape()[1];
  if (vocab == 0 || embd == 0)
    fail(op + ": table " + fmt_shape(table.shape()) + " has a zero axis");
  uint32_t n_tokens = 0;
  const auto &os = out.shape();
  if (os.size() == 1 && os[0] == embd)
    n_tokens = 1;
  else if (os.size() == 2 && os[1] == embd && os[0] > 0)
    n_tokens = os[0];
  else
    fail(op + ": out shape " + fmt_shape(os) + " must be [embd] or [t, embd] with embd=" +
         std::to_string(embd));
  const uint64_t need = (uint64_t)n_tokens * 4;
  if ((uint64_t)tokens.cap() * 4 < need)
    fail(op + ": token buffer " + std::to_string((uint64_t)tokens.cap() * 4) + " B < " +
         std::to_string(need) + " B for " + std::to_string(n_tokens) + " ids");
  if (n_tokens > 65535)
    fail(op + ": " + std::to_string(n_tokens) + " rows exceed the launch grid (65535)");
  EmbedArgs a{};
  a.tokens = reinterpret_cast<const uint32_t *>(tokens.device_address());
  a.table = table.device_ptr();
  a.out = out.device_ptr();
  a.embd = embd;
  a.vocab = vocab;
  a.n_tokens = n_tokens;
  a.table_f16 = table.dtype() == DType::F16;
  a.out_f16 = out.dtype() == DType::F16;
  ElemLaunch l = elem("ta_embed_gather", (embd + 1023) / 1024, a);
  l.gy = n_tokens;
  return l;
}

// ops.rs:243-316 (plan_rope_scatter): f32 input, dst f32 or f16 and not
// the input, every destination element inside dst.
ElemLaunch plan_rope_scatter(ExecutorImpl &e, const Tensor &input, const Tensor &table,
                             const Tensor &dst, const RopeDesc &desc,
                             const RopeScatterDesc &scatter) {
  const std::string op = "run_rope_scatter";
  e.validate_tensor(&input, "input");
  ensure_f32(input, op, "input");
  e.validate_tensor(&table, "table");
  ensure_f32(table, op, "table");
  e.validate_tensor(&dst, "dst");
  if (input.buffer_id() == dst.buffer_id())
    fail(op + ": input and dst must be different tensors");
  const uint64_t tokens = rope_tokens(op, input, table, desc);
  const uint64_t max_index = scatter.dst_offset + (tokens - 1) * scatter.dst_strides[0] +
                             (uint64_t)(desc.heads - 1) * scatter.dst_strides[1] +
                             (uint64_t)(desc.head_dim - 1) * scatter.dst_strides[2];
  if (max_index >= dst.len())
    fail(op + ": destination access reaches element " + std::to_string(max_index) +
         " but dst has " + std::to_string(dst.len()));
  RopeScatterArgs a{};
  a.rope.in = input.device_ptr();
  a.rope.table = static_cast<const float *>(table.device_ptr());
  a.rope.pos_addr = reinterpret_cast<const uint32_t *>(desc.pos_addr);
  a.rope.tokens = (uint32_t)tokens;
  a.rope.heads = desc.heads;
  a.rope.head_dim = desc.head_dim;
  a.rope.rot_dim = desc.rot_dim;
  a.rope.pos_base = desc.pos_base;
  a.rope.table_len = table.len();
  a.dst = dst.device_ptr();
  a.dst_offset = scatter.dst_offset;
  for (int i = 0; i < 3; ++i)
    a.dst_strides[i] = scatter.dst_strides[i];
  a.pos_scale = scatter.pos_scale;
  a.dst_f16 = dst.dtype() == DType::F16;
  a.dst_len = dst.len();
  const uint64_t pairs = tokens * desc.heads * (desc.rot_dim / 2);
  return elem("ta_rope_scatter", grid_for(pairs, 256, e.ctx->cu_count()), a);
}

// ops.rs:318-380 (plan_binary): a, b and out share a storage type and an
// element count; out may alias either input.
ElemLaunch plan_binary(ExecutorImpl &e, const Tensor &a, const Tensor &b, const Tensor &out,
                       BinaryOp bop) {
  const std::string op = "run_binary";
  e.validate_tensor(&a, "a");
  e.validate_tensor(&out, "out");
  const bool f16 = io_f16(op, a, out);
  e.validate_tensor(&b, "b");
  if (b.dtype() != a.dtype())
    fail(op + ": b (" + dtype_name(b.dtype()) + ") must match a (" + dtype_name(a.dtype()) +
         ") storage");
  if (a.len() != b.len() || a.len() != out.len())
    fail(op + ": element counts differ (a " + std::to_string(a.len()) + ", b " +
         std::to_string(b.len()) + ", out " + std::to_string(out.len()) + ")");
  if (a.len() > UINT32_MAX)
    fail(op + ": too large");
  BinaryArgs ba{};
  ba.a = a.device_ptr();
  ba.b = b.device_ptr();
  ba.out = out.device_ptr();
  ba.n = a.len();
  ba.mode = (uint32_t)bop.kind;
  ba.beta = bop.kind == BinaryOp::Kind::AddScaled ? bop.beta : 0.0f;
  ba.io_f16 = f16 ? 1u : 0u;
  return elem("ta_binary", grid_for((a.len() + 3) / 4, 256, e.ctx->cu_count()), ba);
}

// flash.rs:272-402 (plan_prefill_qkv_pack): the same checks in the same
// order.
ElemLaunch plan_prefill_qkv_pack(ExecutorImpl &e, const Tensor &qkv, const Tensor &table,
                                 const Tensor &q, const Tensor &kt, const Tensor &v,
                                 const PrefillQkvPackDesc &d) {
  const std::string op = "run_prefill_qkv_pack";
  for (auto [t, name] : {std::pair<const Tensor *, const char *>{&qkv, "qkv"},
                         {&q, "q"},
                         {&kt, "kt"},
                         {&v, "v"}}) {
    e.validate_tensor(t, name);
    if (t->dtype() != DType::F16)
      fail(op + ": " + name + " must be f16 storage, got " + dtype_name(t->dtype()));
  }
  e.validate_tensor(&table, "table");
  ensure_f32(table, op, "table");
  if (d.heads == 0 || d.kv_heads == 0 || d.head_dim == 0 || d.rot_dim == 0 || d.rot_dim % 2 != 0 ||
      d.rot_dim > d.head_dim)
    fail(op + ": invalid heads/kv_heads/dh/rot_dim (" + std::to_string(d.heads) + "/" +
         std::to_string(d.kv_heads) + "/" + std::to_string(d.head_dim) + "/" +
         std::to_string(d.rot_dim) + ")");
  if (qkv.shape().size() != 2)
    fail(op + ": qkv must be [T, n_qkv], got " + fmt_shape(qkv.shape()));
  const uint32_t tokens = qkv.shape()[0], qkv_stride = qkv.shape()[1];
  const uint64_t embd = (uint64_t)d.heads * d.head_dim, kv_dim = (uint64_t)d.kv_heads * d.head_dim;
  const uint64_t want_stride = embd + 2 * kv_dim;
  if (qkv_stride != want_stride)
    fail(op + ": qkv N " + std::to_string(qkv_stride) + " != H*dh + 2*H_kv*dh (" +
         std::to_string(want_stride) + ")");
  if (q.shape() != std::vector<uint32_t>{d.heads, tokens, d.head_dim})
    fail(op + ": q must be head-major [H=" + std::to_string(d.heads) + ", T=" +
         std::to_string(tokens) + ", dh=" + std::to_string(d.head_dim) + "], got " +
         fmt_shape(q.shape()));
  if (kt.shape().size() != 3)
    fail(op + ": kt must be [H_kv, dh, T_max], got " + fmt_shape(kt.shape()));
  if (v.shape().size() != 3)
    fail(op + ": v must be [H_kv, T_max, dh], got " + fmt_shape(v.shape()));
  const uint32_t t_max = kt.shape()[2];
  if (kt.shape()[0] != d.kv_heads || v.shape()[0] != d.kv_heads || kt.shape()[1] != d.head_dim ||
      v.shape()[2] != d.head_dim || v.shape()[1] != t_max)
    fail(op + ": cache shapes kt " + fmt_shape(kt.shape()) + " v " + fmt_shape(v.shape()) +
         " vs H_kv=" + std::to_string(d.kv_heads) + " dh=" + std::to_string(d.head_dim));
  if ((uint64_t)d.pos_base + tokens > t_max)
    fail(op + ": pos_base " + std::to_string(d.pos_base) + " + T " + std::to_string(tokens) +
         " exceeds T_max " + std::to_string(t_max));
  const uint64_t needed = ((uint64_t)d.pos_base + tokens) * d.rot_dim;
  if (table.len() < needed)
    fail(op + ": table length " + std::to_string(table.len()) + " < required " +
         std::to_string(needed) + " (pos_base " + std::to_string(d.pos_base) + " + " +
         std::to_string(tokens) + " tokens, rot_dim " + std::to_string(d.rot_dim) + ")");
  if (d.head_dim % 4 != 0)
    fail(op + ": head_dim " + std::to_string(d.head_dim) + " must be a multiple of 4");
  QkvPackArgs a{};
  a.qkv = static_cast<const uint16_t *>(qkv.device_ptr());
  a.q = static_cast<uint16_t *>(q.device_ptr());
  a.kt = static_cast<uint16_t *>(kt.device_ptr());
  a.v = static_cast<uint16_t *>(v.device_ptr());
  a.table = static_cast<const float *>(table.device_ptr());
  a.tokens = tokens;
  a.heads = d.heads;
  a.kv_heads = d.kv_heads;
  a.head_dim = d.head_dim;
  a.rot_dim = d.rot_dim;
  a.pos_base = d.pos_base;
  a.qkv_stride = qkv_stride;
  a.t_max = t_max;
  a.k_offset = (uint32_t)embd;
  a.v_offset = (uint32_t)(embd + kv_dim);
  const uint64_t items = (uint64_t)tokens * (d.heads + d.kv_heads) * (d.rot_dim / 2) +
                         (uint64_t)tokens * d.kv_heads * (d.head_dim / 4);
  return elem("ta_prefill_qkv_pack", grid_for(items, 256, e.ctx->cu_count()), a);
}

// Decode-attention chunk count (elementwise/mod.rs:233-241): about 64
// positions (one wave block) per chunk, at least 8 and at most
// kAttnDecodeMaxChunks chunks; position-driven launches always use the cap.
static_assert(kAttnDecodeMaxChunks == TA_ATTN_DECODE_MAX_CHUNKS,
              "the combine kernel's chunk slots and the host cap must agree");
uint32_t attn_decode_num_chunks(uint32_t kv_len) {
  return std::min(kAttnDecodeMaxChunks, std::max(8u, (kv_len + 63) / 64));
}

// attn.rs:61-184 (plan_attn_decode): the same checks in the same order;
// dh 64 and 128 are compiled.
ElemLaunches plan_attn_decode(ExecutorImpl &e, const Tensor &q, const Tensor &kt, const Tensor &v,
                              const Tensor &scratch, const Tensor &out,
                              const AttnDecodeDesc &desc) {
  const std::string op = "run_attn_decode";
  e.validate_tensor(&q, "q");
  ensure_f32(q, op, "q");
  e.validate_tensor(&kt, "kt");
  e.validate_tensor(&v, "v");
  e.validate_tensor(&scratch, "scratch");
  ensure_f32(scratch, op, "scratch");
  e.validate_tensor(&out, "out");
  ensure_f32(out, op, "out");
  if (kt.dtype() != v.dtype())
    fail(op + ": kt (" + dtype_name(kt.dtype()) + ") and v (" + dtype_name(v.dtype()) +
         ") must share a storage type");
  const bool kv16 = kt.dtype() == DType::F16;
  if (kt.shape().size() != 3)
    fail(op + ": kt must be [H_kv, dh, T_max], got " + fmt_shape(kt.shape()));
  if (v.shape().size() != 3)
    fail(op + ": v must be [H_kv, T_max, dh], got " + fmt_shape(v.shape()));
  const uint32_t kv_heads = kt.shape()[0], dh = kt.shape()[1], t_max = kt.shape()[2];
  if (v.shape()[2] != dh || v.shape()[1] != t_max || v.shape()[0] != kv_heads || kv_heads == 0)
    fail(op + ": inconsistent caches kt " + fmt_shape(kt.shape()) + ", v " +
         fmt_shape(v.shape()));
  if (dh != 64 && dh != 128)
    fail(op + ": head dimension " + std::to_string(dh) +
         " unsupported (compiled variants: 64, 128)");
  const uint64_t heads_elems = (uint64_t)kv_heads * dh;
  if (q.len() == 0 || q.len() % heads_elems != 0)
    fail(op + ": q length " + std::to_string(q.len()) + " must be kv_heads*group*dh (kv_heads " +
         std::to_string(kv_heads) + ", dh " + std::to_string(dh) + ")");
  const uint64_t group = q.len() / heads_elems;
  if (group == 0 || group > 8)
    fail(op + ": GQA group " + std::to_string(group) + " unsupported (1..=8)");
  if (out.len() != q.len())
    fail(op + ": out length " + std::to_string(out.len()) + " must equal q length " +
         std::to_string(q.len()));
  if (desc.kv_len == 0 || desc.kv_len > t_max)
    fail(op + ": kv_len " + std::to_string(desc.kv_len) + " out of range 1..=" +
         std::to_string(t_max));
  const uint32_t num_chunks =
      desc.pos_addr ? kAttnDecodeMaxChunks : attn_decode_num_chunks(desc.kv_len);
  if (num_chunks == 0 || num_chunks > TA_ATTN_DECODE_MAX_CHUNKS)
    fail(op + ": internal: " + std::to_string(num_chunks) + " chunks outside 1..=" +
         std::to_string(TA_ATTN_DECODE_MAX_CHUNKS));
  const uint64_t needed = (uint64_t)kv_heads * num_chunks * group * (dh + 2);
  if (scratch.len() < needed)
    fail(op + ": scratch length " + std::to_string(scratch.len()) + " < required " +
         std::to_string(needed) + " (kv_heads " + std::to_string(kv_heads) + " * chunks " +
         std::to_string(num_chunks) + " * group " + std::to_string(group) + " * (dh+2))");
  if (kv_heads > 65535)
    fail(op + ": " + std::to_string(kv_heads) + " kv heads exceed the launch grid (65535)");
  AttnDecodeArgs a{};
  a.q = static_cast<const float *>(q.device_ptr());
  a.kt = kt.device_ptr();
  a.v = v.device_ptr();
  a.scratch = static_cast<float *>(scratch.device_ptr());
  a.pos = reinterpret_cast<const uint32_t *>(desc.pos_addr);
  a.kv_len = desc.kv_len;
  a.num_chunks = num_chunks;
  a.group = (uint32_t)group;
  a.t_max = t_max;
  a.scale = desc.scale;
  const char *sym = kv16 ? (dh == 64 ? "ta_attn_decode_kv16_dh64" : "ta_attn_decode_kv16_dh128")
                         : (dh == 64 ? "ta_attn_decode_dh64" : "ta_attn_decode_dh128");
  ElemLaunch stage1 = elem(sym, num_chunks, a);
  stage1.gy = kv_heads;
  AttnCombineArgs c{};
  c.scratch = a.scratch;
  c.out = static_cast<float *>(out.device_ptr());
  c.num_chunks = num_chunks;
  c.group = (uint32_t)group;
  c.dh = dh;
  ElemLaunch combine = elem("ta_attn_decode_combine", (uint32_t)(kv_heads * group), c);
  combine.threads = 64;
  return {stage1, combine};
}
} // namespace

// gemv_chain.rs:17-45 and 106-179 (plan_gemv_chain, pack_gemv_job): the
// same job rules and messages.
void check_gemv_chain(const ExecutorImpl &e, const std::vector<MatmulOp> &jobs) {
  if (jobs.empty())
    fail("gemv_chain: empty job list");
  if (jobs.size() > kGemvChainMaxJobs)
    fail("gemv_chain: " + std::to_string(jobs.size()) + " jobs exceeds max " +
         std::to_string(kGemvChainMaxJobs));
  for (size_t i = 0; i < jobs.size(); ++i) {
    const MatmulOp &op = jobs[i];
    const std::string at = "gemv_chain[" + std::to_string(i) + "]: ";
    e.validate_op(op);
    if (!op.store.is_none())
      fail(at + "fused store epilogues are not supported");
    if (op.call.accumulate)
      fail(at + "accumulate is not supported");
    if (op.call.a->dtype() != DType::F32 || op.call.c->dtype() != DType::F32)
      fail(at + "A and C must be f32 storage");
    if (op.call.b->dtype() != DType::F16)
      fail(at + "B must be f16 storage");
    if (op.packed_b)
      fail(at + "packed-B layout is not supported");
    if (op.epilogue.bias)
      fail(at + "bias epilogue is not supported");
    const ResolvedMatmul d = ResolvedMatmul::from_op(op);
    if (d.batch != 1 || d.m != 1)
      fail(at + "requires batch=1 M=1 (got B=" + std::to_string(d.batch) + " M=" +
           std::to_string(d.m) + ")");
    if (op.epilogue.activation != Activation::None && op.epilogue.activation != Activation::Silu)
      fail(at + "unsupported activation " + std::to_string((uint32_t)op.epilogue.activation));
    if (op.normed_a && op.epilogue.binary.kind == EpilogueBinary::Kind::AddScaled)
      fail(at + "NORM_A cannot combine with AddScaled");
  }
}

ElemLaunches plan_exec_elem(ExecutorImpl &e, const ExecOp &op) {
  auto need = [&](const Tensor *t, const char *role) -> const Tensor & {
    if (!t)
      fail(std::string("run_exec_ops: ") + role + " tensor is null");
    return *t;
  };
  switch (op.kind) {
  case ExecOp::Kind::RmsNorm:
    return {plan_norm(e, "run_rms_norm", need(op.in[0], "input"), need(op.in[1], "weight"),
                     nullptr, need(op.out, "output"), op.scalar)};
  case ExecOp::Kind::LayerNorm:
    return {plan_norm(e, "run_layer_norm", need(op.in[0], "input"), need(op.in[1], "weight"),
                     &need(op.in[2], "bias"), need(op.out, "output"), op.scalar)};
  case ExecOp::Kind::SoftmaxRows:
    return {plan_softmax(e, need(op.in[0], "input"), need(op.out, "output"), op.scalar, op.mask)};
  case ExecOp::Kind::Rope:
    return {plan_rope(e, need(op.in[0], "input"), need(op.in[1], "table"), need(op.out, "output"),
                     op.rope)};
  case ExecOp::Kind::CopyStrided:
    return {plan_copy(e, need(op.in[0], "src"), need(op.out, "dst"), op.copy)};
  case ExecOp::Kind::FlashAttn:
    return {plan_flash(e, need(op.in[0], "q"), need(op.in[1], "kt"), need(op.in[2], "v"),
                      need(op.out, "out"), op.flash)};
  case ExecOp::Kind::Argmax:
    if (!op.cell)
      fail("run_exec_ops: result cell is null");
    return {plan_argmax(e, need(op.in[0], "input"), *op.cell)};
  case ExecOp::Kind::EmbedGather:
    if (!op.cell)
      fail("run_exec_ops: token cell is null");
    return {plan_embed_gather(e, *op.cell, need(op.in[0], "table"), need(op.out, "out"))};
  case ExecOp::Kind::AttnDecode:
    return plan_attn_decode(e, need(op.in[0], "q"), need(op.in[1], "kt"), need(op.in[2], "v"),
                            need(op.aux, "scratch"), need(op.out, "out"), op.attn);
  case ExecOp::Kind::RopeScatter:
    return {plan_rope_scatter(e, need(op.in[0], "input"), need(op.in[1], "table"),
                              need(op.out, "dst"), op.rope, op.scatter)};
  case ExecOp::Kind::Binary:
    return {plan_binary(e, need(op.in[0], "a"), need(op.in[1], "b"), need(op.out, "out"),
                        op.binary)};
  case ExecOp::Kind::PrefillQkvPack:
    return {plan_prefill_qkv_pack(e, need(op.in[0], "qkv"), need(op.in[1], "table"),
                                  need(op.out, "q"), need(op.aux, "kt"), need(op.aux2, "v"),
                                  op.qkv)};
  case ExecOp::Kind::Matmul:
  case ExecOp::Kind::GemvChain:
    break;
  }
  fail("internal: plan_exec_elem on a matmul step");
}

RunStats Executor::run_softmax_rows(const Tensor &input, const Tensor &output, float scale,
                                    SoftmaxMask mask) const {
  return impl_->run_elem(plan_softmax(*impl_, input, output, scale, mask));
}
RunStats Executor::run_rms_norm(const Tensor &input, const Tensor &weight, const Tensor &output,
                                float eps) const {
  return impl_->run_elem(plan_norm(*impl_, "run_rms_norm", input, weight, nullptr, output, eps));
}
RunStats Executor::run_layer_norm(const Tensor &input, const Tensor &weight, const Tensor &bias,
                                  const Tensor &output, float eps) const {
  return impl_->run_elem(plan_norm(*impl_, "run_layer_norm", input, weight, &bias, output, eps));
}
RunStats Executor::run_rope(const Tensor &input, const Tensor &table, const Tensor &output,
                            const RopeDesc &desc) const {
  return impl_->run_elem(plan_rope(*impl_, input, table, output, desc));
}
RunStats Executor::run_copy_strided(const Tensor &src, const Tensor &dst,
                                    const CopyDesc &desc) const {
  return impl_->run_elem(plan_copy(*impl_, src, dst, desc));
}
RunStats Executor::run_flash_attention(const Tensor &q, const Tensor &kt, const Tensor &v,
                                       const Tensor &out, const FlashAttentionDesc &desc) const {
  return impl_->run_elem(plan_flash(*impl_, q, kt, v, out, desc));
}
RunStats Executor::run_rope_scatter(const Tensor &input, const Tensor &table, const Tensor &dst,
                                    const RopeDesc &desc, const RopeScatterDesc &scatter) const {
  return impl_->run_elem(plan_rope_scatter(*impl_, input, table, dst, desc, scatter));
}
RunStats Executor::run_binary(const Tensor &a, const Tensor &b, const Tensor &out,
                              BinaryOp op) const {
  return impl_->run_elem(plan_binary(*impl_, a, b, out, op));
}
RunStats Executor::run_prefill_qkv_pack(const Tensor &qkv, const Tensor &table, const Tensor &q,
                                        const Tensor &kt, const Tensor &v,
                                        const PrefillQkvPackDesc &desc) const {
  return impl_->run_elem(plan_prefill_qkv_pack(*impl_, qkv, table, q, kt, v, desc));
}
RunStats Executor::run_argmax(const Tensor &input, const U32Cell &result) const {
  return impl_->run_elem(plan_argmax(*impl_, input, result));
}
RunStats Executor::run_embed_gather(const U32Cell &tokens, const Tensor &table,
                                    const Tensor &out) const {
  return impl_->run_elem(plan_embed_gather(*impl_, tokens, table, out));
}
RunStats Executor::run_attn_decode(const Tensor &q, const Tensor &kt, const Tensor &v,
                                   const Tensor &scratch, const Tensor &out,
                                   const AttnDecodeDesc &desc) const {
  return impl_->run_elem(plan_attn_decode(*impl_, q, kt, v, scratch, out, desc));
}
RunStats Executor::run_exec_ops(const std::vector<ExecOp> &ops) const {
  return impl_->run_exec_impl(ops);
}
std::unique_ptr<PreparedOps> Executor::prepare_exec_ops(const std::vector<ExecOp> &ops) const {
  return impl_->prepare_exec_impl(this, ops);
}

std::unique_ptr<PreparedOps> Executor::prepare_matmuls(const std::vector<MatmulCall> &calls) const {
  std::vector<MatmulOp> ops;
  for (const auto &c : calls)
    ops.emplace_back(c);
  return impl_->prepare_impl(this, ops, false);
}
std::unique_ptr<PreparedOps> Executor::prepare_ops(const std::vector<MatmulOp> &ops) const {
  return impl_->prepare_impl(this, ops, false);
}
std::unique_ptr<PreparedOps> Executor::prepare_op_graph(const std::vector<MatmulOp> &ops) const {
  return impl_->prepare_impl(this, ops, true);
}

// src/executor/tuning.rs:18-56: tune against 1.0-filled scratch tensors.
void Executor::tune_shape(uint32_t batch, uint32_t m, uint32_t n, uint32_t k) const {
  const TuneKey key{batch, m, n, k, false};
  if (impl_->is_tuned(key))
    return;
  impl_->ctx->make_current();
  auto shape = [&](uint32_t r, uint32_t c) {
    return batch == 1 ? std::vector<uint32_t>{r, c} : std::vector<uint32_t>{batch, r, c};
  };
  Tensor a = Tensor::uninit_device(impl_->ctx, shape(m, k));
  Tensor b = Tensor::uninit_device(impl_->ctx, shape(k, n));
  Tensor c = Tensor::uninit_device(impl_->ctx, shape(m, n));
  std::vector<float> ones(std::max(a.len(), b.len()), 1.0f);
  upload(ones.data(), a.len(), a);
  upload(ones.data(), b.len(), b);
  MatmulOp op(MatmulCall{&a, &b, &c, 1.0f, false});
  ResolvedMatmul d = ResolvedMatmul::from_op(op);
  impl_->tune_op(op, d);
}

DispatchInfo Executor::dispatch_info(uint32_t batch, uint32_t m, uint32_t n, uint32_t k) const {
  return dispatch_info_for(batch, m, n, k, false);
}

// src/executor/mod.rs:156-172.
DispatchInfo Executor::dispatch_info_for(uint32_t batch, uint32_t m, uint32_t n, uint32_t k,
                                         bool b_f16) const {
  OpPlan p = impl_->plan_shape(batch, m, n, k, b_f16, true);
  const KernelSpec &s = p.splitk2 ? splitk_stage1_spec(m, n, k) : KERNEL_SPECS[p.kernel];
  DispatchInfo info;
  info.kernel = s.name;
  info.tile = {s.tile_m, s.tile_n, s.tile_k};
  info.split_k2_splits = p.splitk2;
  return info;
}

void Executor::upload(const float *src, size_t len, const Tensor &dst) const {
  impl_->validate_tensor(&dst, "upload destination");
  if (len == 0)
    return;
  impl_->ctx->make_current();
  if (dst.dtype() == DType::F32) {
    impl_->copy_to_device(src, (uint64_t)len * 4, dst, "upload");
  } else {
    std::vector<uint16_t> halves(len);
    for (size_t i = 0; i < len; ++i)
      halves[i] = f32_to_f16_bits(src[i]);
    impl_->copy_to_device(halves.data(), (uint64_t)len * 2, dst, "upload");
  }
}

void Executor::upload_f16(const uint16_t *src, size_t len, const Tensor &dst) const {
  impl_->validate_tensor(&dst, "upload destination");
  if (len == 0)
    return;
  if (dst.dtype() != DType::F16)
    fail(std::string("upload_f16 requires an f16 destination tensor, got ") +
         dtype_name(dst.dtype()));
  impl_->ctx->make_current();
  impl_->copy_to_device(src, (uint64_t)len * 2, dst, "upload");
}

void Executor::download(const Tensor &src, float *dst, size_t len) const {
  impl_->validate_tensor(&src, "download source");
  if (len == 0)
    return;
  impl_->ctx->make_current();
  const uint64_t bytes = (uint64_t)len * dtype_size(src.dtype());
  if (bytes > src.size_bytes())
    fail("download: " + std::to_string(bytes) + " bytes > tensor capacity " +
         std::to_string(src.size_bytes()));
  ExecutorImpl::Lease lease(impl_.get());
  if (src.dtype() == DType::F32) {
    hip_check(hipMemcpyAsync(dst, src.device_ptr(), bytes, hipMemcpyDeviceToHost, lease.s->stream),
              "hipMemcpyAsync (download)");
    hip_check(hipStreamSynchronize(lease.s->stream), "hipStreamSynchronize");
  } else {
    std::vector<uint16_t> halves(len);
    hip_check(hipMemcpyAsync(halves.data(), src.device_ptr(), bytes, hipMemcpyDeviceToHost,
                             lease.s->stream),
              "hipMemcpyAsync (download)");
    hip_check(hipStreamSynchronize(lease.s->stream), "hipStreamSynchronize");
    for (size_t i = 0; i < len; ++i)
      dst[i] = f16_bits_to_f32(halves[i]);
  }
}

// ------------------------------------------------------------ PreparedOps

PreparedOps::~PreparedOps() {
  if (!exec_)
    return;
  (void)hipSetDevice(exec_->context()->device());
  hipStream_t s = static_cast<hipStream_t>(stream_);
  if (s)
    (void)hipStreamSynchronize(s); // Drop waits for in-flight work
  if (graph_exec_)
    (void)hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec_));
  for (void *p : scratch_)
    if (p)
      (void)hipFree(p);
  if (ev_start_)
    (void)hipEventDestroy(static_cast<hipEvent_t>(ev_start_));
  if (ev_end_)
    (void)hipEventDestroy(static_cast<hipEvent_t>(ev_end_));
  if (status_)
    (void)hipHostFree(status_);
  if (s)
    (void)hipStreamDestroy(s);
}

RunStats PreparedOps::run() {
  submit();
  return wait();
}

void PreparedOps::run_silent() {
  submit();
  hip_check(hipStreamSynchronize(static_cast<hipStream_t>(stream_)), "hipStreamSynchronize");
  in_flight_ = false;
  if (status_)
    check_host_status(static_cast<uint32_t *>(status_), mlp_scratch_, mlp_bytes_);
}

// src/executor/prepared.rs:293-307.
void PreparedOps::submit() {
  if (in_flight_)
    fail("PreparedOps::submit: already in flight; call wait() first");
  exec_->context()->make_current();
  hipStream_t s = static_cast<hipStream_t>(stream_);
  hip_check(hipEventRecord(static_cast<hipEvent_t>(ev_start_), s), "hipEventRecord");
  hip_check(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec_), s), "hipGraphLaunch");
  hip_check(hipEventRecord(static_cast<hipEvent_t>(ev_end_), s), "hipEventRecord");
  in_flight_ = true;
  submitted_once_ = true;
}

RunStats PreparedOps::wait() {
  if (!in_flight_)
    fail("PreparedOps::wait: nothing submitted");
  exec_->context()->make_current();
  hip_check(hipEventSynchronize(static_cast<hipEvent_t>(ev_end_)), "hipEventSynchronize");
  in_flight_ = false;
  float ms = 0.f;
  hip_check(hipEventElapsedTime(&ms, static_cast<hipEvent_t>(ev_start_),
                                static_cast<hipEvent_t>(ev_end_)),
            "hipEventElapsedTime");
  if (status_)
    check_host_status(static_cast<uint32_t *>(status_), mlp_scratch_, mlp_bytes_);
  return RunStats{(uint64_t)((double)ms * 1e6), n_calls_, flops_};
}

} // namespace tensor_ash
