// C++ mirror of the reference's Rust API for the fused-epilogue GEMM path
// (gusahlg/tensor-ash: src/lib.rs re-exports).  Same type and function
// names, argument meaning and error behaviour (errors are thrown as
// tensor_ash::Error with the reference's message text).  The C ABI in
// include/tensor_ash.h is a thin layer over this header.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

namespace tensor_ash {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// src/dtype.rs:10-18.
enum class DType { F32, F16 };
uint64_t dtype_size(DType d);
const char *dtype_name(DType d);

// src/dtype.rs:42-112 (f16 decode is exact IEEE, see dtype.cpp).
uint16_t f32_to_f16_bits(float value);
float f16_bits_to_f32(uint16_t bits);
float round_f32_via_f16(float value);

class Context;
struct DeviceBuffer;

// src/tensor.rs:20-174: shape + dtype + shared device allocation.
class Tensor {
public:
  static Tensor uninit_device(const std::shared_ptr<Context> &ctx,
                              const std::vector<uint32_t> &shape);
  static Tensor uninit_device_f16(const std::shared_ptr<Context> &ctx,
                                  const std::vector<uint32_t> &shape);
  static uint64_t numel_checked(const std::vector<uint32_t> &shape);

  Tensor alias_with_shape(const std::vector<uint32_t> &shape) const;
  const std::vector<uint32_t> &shape() const { return shape_; }
  DType dtype() const { return dtype_; }
  uint64_t len() const;
  uint64_t size_bytes() const;
  void *device_ptr() const;
  const DeviceBuffer *buffer_id() const { return buffer_.get(); }
  bool belongs_to(const Context *ctx) const;

private:
  Tensor(std::vector<uint32_t> shape, DType dtype, std::shared_ptr<DeviceBuffer> buf)
      : shape_(std::move(shape)), dtype_(dtype), buffer_(std::move(buf)) {}
  std::vector<uint32_t> shape_;
  DType dtype_;
  std::shared_ptr<DeviceBuffer> buffer_;
};

// src/matmul/api.rs:5-11.
struct MatmulCall {
  const Tensor *a = nullptr;
  const Tensor *b = nullptr;
  const Tensor *c = nullptr;
  float alpha = 1.0f;
  bool accumulate = false;
};

// src/matmul/api.rs:15-35 (codes 0-3).
enum class Activation : uint32_t { None = 0, Relu = 1, Silu = 2, Gelu = 3 };

// src/matmul/api.rs:41-48.
struct EpilogueBinary {
  enum class Kind : uint32_t { None = 0, AddScaled = 1, Mul = 2 };
  Kind kind = Kind::None;
  const Tensor *d = nullptr;
  float beta = 0.0f;
  static EpilogueBinary none() { return {}; }
  static EpilogueBinary add_scaled(const Tensor &d, float beta) {
    return {Kind::AddScaled, &d, beta};
  }
  static EpilogueBinary mul(const Tensor &d) { return {Kind::Mul, &d, 0.0f}; }
};

// src/matmul/api.rs:56-105.
struct Epilogue {
  const Tensor *bias = nullptr;
  Activation activation = Activation::None;
  EpilogueBinary binary;
  bool is_none() const {
    return bias == nullptr && activation == Activation::None &&
           binary.kind == EpilogueBinary::Kind::None;
  }
  const Tensor *d_tensor() const {
    return binary.kind == EpilogueBinary::Kind::None ? nullptr : binary.d;
  }
};

// src/matmul/api.rs:107-133: geometry of the fused store epilogue.  The
// position is P = pos_base + *pos_addr (pos_addr: device address of a u32
// cell, 0 = none); output column c scatters to element
// P * pos_scale + (c / head_dim) * stride_head + (c % head_dim) * stride_dim;
// RoPE rotates the interleaved (even, odd) pairs of each head by the
// (cos, sin) at row P * head_dim/2 + (c % head_dim)/2 of a
// [T_max, head_dim/2, 2] f32 table.
struct MatmulStoreDesc {
  uint32_t head_dim = 0;
  uint32_t pos_base = 0;
  uint32_t pos_scale = 0;
  uint32_t stride_head = 0;
  uint32_t stride_dim = 0;
  uint64_t pos_addr = 0;
};

// src/matmul/api.rs:135-206: fused store-time destination of an M = 1
// f16-weights decode GEMV (codes are the reference's STORE_MODE values).
struct MatmulStore {
  enum class Kind : uint32_t { None = 0, Rope = 1, Scatter = 2, RopeScatter = 3 };
  Kind kind = Kind::None;
  const Tensor *table = nullptr; // Rope, RopeScatter
  const Tensor *dst = nullptr;   // Scatter, RopeScatter (f32 or f16)
  MatmulStoreDesc desc;
  bool is_none() const { return kind == Kind::None; }
  uint32_t mode() const { return (uint32_t)kind; }
};

// src/matmul/api.rs:213-299.  normed_a = (weight, eps): C = rms_norm(A,
// weight, eps) @ B, on the decode GEMV routes only.
struct NormedA {
  const Tensor *weight = nullptr;
  float eps = 0.0f;
};

struct MatmulOp {
  MatmulCall call;
  Epilogue epilogue;
  std::optional<NormedA> normed_a;
  MatmulStore store;
  bool packed_b = false;
  MatmulOp() = default;
  explicit MatmulOp(const MatmulCall &c) : call(c) {}
  MatmulOp(const MatmulCall &c, const Epilogue &e) : call(c), epilogue(e) {}
  static MatmulOp with_epilogue(const MatmulCall &c, const Epilogue &e) {
    return MatmulOp(c, e);
  }
  MatmulOp with_packed_b() const {
    MatmulOp o = *this;
    o.packed_b = true;
    return o;
  }
  MatmulOp with_normed_a(const Tensor &weight, float eps) const {
    MatmulOp o = *this;
    o.normed_a = NormedA{&weight, eps};
    return o;
  }
  MatmulOp with_store_rope(const Tensor &table, const MatmulStoreDesc &desc) const {
    MatmulOp o = *this;
    o.store = MatmulStore{MatmulStore::Kind::Rope, &table, nullptr, desc};
    return o;
  }
  MatmulOp with_store_scatter(const Tensor &dst, const MatmulStoreDesc &desc) const {
    MatmulOp o = *this;
    o.store = MatmulStore{MatmulStore::Kind::Scatter, nullptr, &dst, desc};
    return o;
  }
  MatmulOp with_store_rope_scatter(const Tensor &table, const Tensor &dst,
                                   const MatmulStoreDesc &desc) const {
    MatmulOp o = *this;
    o.store = MatmulStore{MatmulStore::Kind::RopeScatter, &table, &dst, desc};
    return o;
  }
  bool has_decode_fusion() const { return normed_a.has_value() || !store.is_none(); }
};

// Model-op descriptors (src/executor/elementwise/mod.rs:112-270).
struct SoftmaxMask {
  enum class Kind { Full, Prefix, Causal };
  Kind kind = Kind::Full;
  uint32_t valid = 0;          // Prefix
  uint32_t prefix = 0;         // Causal
  uint32_t rows_per_group = 0; // Causal
  static SoftmaxMask full() { return {}; }
  static SoftmaxMask prefix_of(uint32_t valid) { return {Kind::Prefix, valid, 0, 0}; }
  static SoftmaxMask causal(uint32_t prefix, uint32_t rows_per_group) {
    return {Kind::Causal, 0, prefix, rows_per_group};
  }
};
struct RopeDesc {
  uint32_t heads = 0, head_dim = 0, rot_dim = 0, pos_base = 0;
  uint64_t pos_addr = 0; // device address of a u32 position, 0 = none
};
// Destination of the fused RoPE + scatter (elementwise/mod.rs:144-159):
// element (token, head, dim) goes to dst_offset (+ *pos_addr * pos_scale
// when the RopeDesc has a position cell) + token * dst_strides[0] + head *
// dst_strides[1] + dim * dst_strides[2].
struct RopeScatterDesc {
  uint32_t dst_offset = 0;
  std::array<uint32_t, 3> dst_strides{};
  uint32_t pos_scale = 0;
};
// Standalone binary combine (elementwise/mod.rs:242-252): out = a + beta *
// b, or out = silu(a) * b.
struct BinaryOp {
  enum class Kind : uint32_t { AddScaled = 0, SiluMul = 1 };
  Kind kind = Kind::AddScaled;
  float beta = 0.0f;
  static BinaryOp add_scaled(float beta) { return {Kind::AddScaled, beta}; }
  static BinaryOp silu_mul() { return {Kind::SiluMul, 0.0f}; }
};
// Prefill QKV pack geometry (elementwise/mod.rs:186-199).
struct PrefillQkvPackDesc {
  uint32_t heads = 0, kv_heads = 0, head_dim = 0;
  uint32_t rot_dim = 0; // even, <= head_dim; lanes past it pass through
  uint32_t pos_base = 0; // absolute position of token 0
};
struct CopyDesc {
  std::array<uint32_t, 3> extent{};
  uint32_t src_offset = 0;
  std::array<uint32_t, 3> src_strides{};
  uint32_t dst_offset = 0;
  std::array<uint32_t, 3> dst_strides{};
  uint64_t pos_addr = 0; // device address of a u32 position, 0 = none
  uint32_t pos_scale = 0;
};

// Causal prefill attention geometry (src/executor/elementwise/mod.rs:
// 160-184).  q/out default to head-major [H, T_q, dh]; token_major_heads
// = H reads q (and, unless out_token_major_heads says otherwise, writes
// out) as token-major [T, H*dh] / [T, H, dh].
struct FlashAttentionDesc {
  uint32_t kv_len = 0;   // valid cache positions
  uint32_t pos_base = 0; // absolute position of query row 0
  float scale = 1.0f;    // 1/sqrt(dh) for standard attention
  std::optional<uint32_t> token_major_heads;
  std::optional<uint32_t> out_token_major_heads;
};

// Fused split-K decode attention geometry (src/executor/elementwise/mod.rs:
// 200-227): one query row per head attends to the kv_len valid cache
// positions.  pos_addr (device address of a u32 cell, 0 = none) makes the
// effective length kv_len + *pos_addr, read at execution time, and fixes
// the chunk count at kAttnDecodeMaxChunks.
struct AttnDecodeDesc {
  uint32_t kv_len = 0;
  float scale = 1.0f;
  uint64_t pos_addr = 0;
};
// Jobs of one run_gemv_chain (elementwise/mod.rs GEMV_CHAIN_MAX_JOBS).
constexpr size_t kGemvChainMaxJobs = 8;
// Chunk bound of decode attention; sizes its scratch: kv_heads *
// kAttnDecodeMaxChunks * group * (dh + 2) f32 (elementwise/mod.rs:229-232).
constexpr uint32_t kAttnDecodeMaxChunks = 32;

class Context;

// Host-visible u32 cells (src/executor/cells.rs:10-205): pinned, mapped
// host memory that kernels read and write through device_address() and
// the host through write()/read() between submissions.  One type serves
// the reference's PosBuffer and HostU32Buffer (cap 1) and TokenIdBuffer
// (cap ids).
class U32Cell {
public:
  static std::unique_ptr<U32Cell> create(const std::shared_ptr<Context> &ctx, uint32_t cap);
  ~U32Cell();
  U32Cell(const U32Cell &) = delete;
  U32Cell &operator=(const U32Cell &) = delete;
  void set(uint32_t value) { write(&value, 1); }
  void write(const uint32_t *values, size_t n);
  uint32_t read() const; // element 0, after the writing submission completed
  uint64_t device_address() const { return device_; }
  uint32_t cap() const { return cap_; }
  const Context *context() const { return ctx_.get(); }

private:
  U32Cell() = default;
  std::shared_ptr<Context> ctx_;
  uint32_t *host_ = nullptr;
  uint64_t device_ = 0;
  uint32_t cap_ = 0;
};

// One step of a mixed-op graph (src/executor/graph_ops.rs:23-171): ops run
// in list order and each sees every earlier op's writes.  Operand roles:
//   Matmul      `matmul`
//   RmsNorm     in[0] input, in[1] weight, out output, scalar eps
//   LayerNorm   in[0] input, in[1] weight, in[2] bias, out, scalar eps
//   SoftmaxRows in[0] input, out, scalar scale, mask
//   Rope        in[0] input, in[1] table, out, rope
//   CopyStrided in[0] src, out dst, copy
//   FlashAttn   in[0] q, in[1] kt, in[2] v, out, flash
//   Argmax      in[0] input, cell result
//   EmbedGather cell token ids, in[0] table, out
//   AttnDecode  in[0] q, in[1] kt, in[2] v, aux scratch, out, attn
//   RopeScatter in[0] input, in[1] table, out dst, rope, scatter
//   Binary      in[0] a, in[1] b, out, binary
//   PrefillQkvPack in[0] qkv, in[1] table, out q, aux kt, aux2 v, qkv
//   GemvChain   jobs (run_gemv_chain's rules)
struct ExecOp {
  enum class Kind {
    Matmul,
    RmsNorm,
    LayerNorm,
    SoftmaxRows,
    Rope,
    CopyStrided,
    FlashAttn,
    Argmax,
    EmbedGather,
    AttnDecode,
    RopeScatter,
    Binary,
    PrefillQkvPack,
    GemvChain
  };
  Kind kind = Kind::Matmul;
  MatmulOp matmul;
  std::vector<MatmulOp> jobs;
  std::array<const Tensor *, 3> in{};
  const Tensor *out = nullptr;
  const Tensor *aux = nullptr;
  const Tensor *aux2 = nullptr;
  const U32Cell *cell = nullptr;
  float scalar = 0.0f;
  SoftmaxMask mask;
  RopeDesc rope;
  CopyDesc copy;
  FlashAttentionDesc flash;
  AttnDecodeDesc attn;
  RopeScatterDesc scatter;
  BinaryOp binary;
  PrefillQkvPackDesc qkv;

  static ExecOp from_matmul(const MatmulOp &op) {
    ExecOp e;
    e.matmul = op;
    return e;
  }
  static ExecOp rms_norm(const Tensor &input, const Tensor &weight, const Tensor &output,
                         float eps) {
    return make(Kind::RmsNorm, {&input, &weight, nullptr}, &output, eps);
  }
  static ExecOp layer_norm(const Tensor &input, const Tensor &weight, const Tensor &bias,
                           const Tensor &output, float eps) {
    return make(Kind::LayerNorm, {&input, &weight, &bias}, &output, eps);
  }
  static ExecOp softmax_rows(const Tensor &input, const Tensor &output, float scale,
                             SoftmaxMask mask) {
    ExecOp e = make(Kind::SoftmaxRows, {&input, nullptr, nullptr}, &output, scale);
    e.mask = mask;
    return e;
  }
  static ExecOp rope_op(const Tensor &input, const Tensor &table, const Tensor &output,
                        const RopeDesc &desc) {
    ExecOp e = make(Kind::Rope, {&input, &table, nullptr}, &output, 0.0f);
    e.rope = desc;
    return e;
  }
  static ExecOp copy_strided(const Tensor &src, const Tensor &dst, const CopyDesc &desc) {
    ExecOp e = make(Kind::CopyStrided, {&src, nullptr, nullptr}, &dst, 0.0f);
    e.copy = desc;
    return e;
  }
  static ExecOp flash_attn(const Tensor &q, const Tensor &kt, const Tensor &v, const Tensor &out,
                           const FlashAttentionDesc &desc) {
    ExecOp e = make(Kind::FlashAttn, {&q, &kt, &v}, &out, 0.0f);
    e.flash = desc;
    return e;
  }

  static ExecOp gemv_chain(const std::vector<MatmulOp> &jobs) {
    ExecOp e;
    e.kind = Kind::GemvChain;
    e.jobs = jobs;
    return e;
  }
  static ExecOp argmax(const Tensor &input, const U32Cell &result) {
    ExecOp e = make(Kind::Argmax, {&input, nullptr, nullptr}, nullptr, 0.0f);
    e.cell = &result;
    return e;
  }
  static ExecOp embed_gather(const U32Cell &tokens, const Tensor &table, const Tensor &out) {
    ExecOp e = make(Kind::EmbedGather, {&table, nullptr, nullptr}, &out, 0.0f);
    e.cell = &tokens;
    return e;
  }
  static ExecOp rope_scatter(const Tensor &input, const Tensor &table, const Tensor &dst,
                             const RopeDesc &desc, const RopeScatterDesc &scatter) {
    ExecOp e = make(Kind::RopeScatter, {&input, &table, nullptr}, &dst, 0.0f);
    e.rope = desc;
    e.scatter = scatter;
    return e;
  }
  static ExecOp binary_op(const Tensor &a, const Tensor &b, const Tensor &out, BinaryOp op) {
    ExecOp e = make(Kind::Binary, {&a, &b, nullptr}, &out, 0.0f);
    e.binary = op;
    return e;
  }
  static ExecOp prefill_qkv_pack(const Tensor &qkv, const Tensor &table, const Tensor &q,
                                 const Tensor &kt, const Tensor &v,
                                 const PrefillQkvPackDesc &desc) {
    ExecOp e = make(Kind::PrefillQkvPack, {&qkv, &table, nullptr}, &q, 0.0f);
    e.aux = &kt;
    e.aux2 = &v;
    e.qkv = desc;
    return e;
  }
  static ExecOp attn_decode(const Tensor &q, const Tensor &kt, const Tensor &v,
                            const Tensor &scratch, const Tensor &out, const AttnDecodeDesc &desc) {
    ExecOp e = make(Kind::AttnDecode, {&q, &kt, &v}, &out, 0.0f);
    e.aux = &scratch;
    e.attn = desc;
    return e;
  }

private:
  static ExecOp make(Kind k, std::array<const Tensor *, 3> in, const Tensor *out, float scalar) {
    ExecOp e;
    e.kind = k;
    e.in = in;
    e.out = out;
    e.scalar = scalar;
    return e;
  }
};

// src/matmul/api.rs:311-353.
struct RunStats {
  std::optional<uint64_t> gpu_time_ns;
  size_t n_calls = 0;
  uint64_t total_flops = 0;
  std::optional<double> tflops() const {
    if (!gpu_time_ns || *gpu_time_ns == 0)
      return std::nullopt;
    return (double)total_flops / (double)*gpu_time_ns * 1e-3;
  }
};

// src/executor/mod.rs:64-81.
struct DispatchInfo {
  const char *kernel = "";
  std::array<uint32_t, 3> tile{0, 0, 0};
  std::optional<uint32_t> split_k2_splits;
};

// src/executor/mod.rs:86-100.
struct ExecutorConfig {
  size_t n_slots = 2;
  uint32_t max_calls_per_submit = 64;
  bool tune = false;
};

// src/matmul/api.rs:324-344 and src/pipeline/routing.rs:10-23.
std::vector<float> pack_f16w_row_tiles(const float *src, size_t k, size_t n, size_t tile_n);
uint32_t f16w_row_tile_n(uint32_t k, uint32_t n);

// src/pipeline/catalog.rs:10-197: one registry entry per gfx950 kernel.
enum class KernelKind : uint32_t {
  GemmF32,       // f32 A, f32 B, FP32 MFMA
  GemmF16w,      // f32 A, f16 B widened to f32, FP32 MFMA
  GemmF16Mfma,   // f32 A rounded to f16, f16 B, f16 MFMA, f32 accumulation
  GemmA16,       // f16 A, f16 B, f16 C (RNE store), f16 MFMA
  GemmF16Sk,     // f32 A rounded to f16 at fragment read, f16 B, f16 MFMA, split-K in the launch
  GemvF16Packed, // M <= 8 decode GEMV, f16 B packed [N/TW][K][TW]
  GemvF16Row,    // M <= 8 decode GEMV, f16 B row-major
  GemvF32Row,    // M <= 8 decode GEMV, f32 B row-major
};
struct KernelSpec {
  const char *name;
  uint32_t tile_m, tile_n, tile_k;
  KernelKind kind;
  const char *symbol; // code-object symbol stem
  const char *aliases; // extra ML_KERNEL spellings, comma separated
  bool weights_f16() const {
    return kind == KernelKind::GemmF16w || kind == KernelKind::GemmF16Mfma ||
           kind == KernelKind::GemmA16 || kind == KernelKind::GemmF16Sk ||
           kind == KernelKind::GemvF16Packed ||
           kind == KernelKind::GemvF16Row;
  }
  bool is_gemv() const {
    return kind == KernelKind::GemvF16Packed || kind == KernelKind::GemvF16Row ||
           kind == KernelKind::GemvF32Row;
  }
  bool packed() const { return kind == KernelKind::GemvF16Packed; }
  // src/pipeline/runtime.rs:62-76: the decode GEMVs implement the fused
  // normed-A preamble; the f16-weight ones also the store epilogue.
  bool supports_normed_a() const { return is_gemv(); }
  bool supports_store() const { return is_gemv() && weights_f16(); }
};
extern const KernelSpec KERNEL_SPECS[];
extern const size_t KERNEL_SPECS_LEN;

// ML_KERNEL value: Auto or one registry index.
struct KernelSelection {
  std::optional<size_t> index; // nullopt = Auto
  static KernelSelection parse(const std::string &value);
  static KernelSelection from_env();
  bool is_auto() const { return !index.has_value(); }
};

// src/context: one HIP device + the loaded gfx950 code objects.
class Context {
public:
  // preference: "auto", "discrete", "index:N", "N", "name:<substr>",
  // "<substr>" (src/context/device.rs:18-54).
  static std::shared_ptr<Context> create(bool enable_validation,
                                         const std::string &preference);
  ~Context();
  int device() const { return device_; }
  uint32_t cu_count() const { return cu_count_; }
  const std::string &device_name() const { return name_; }
  const std::string &arch() const { return arch_; }
  int runtime_version() const { return runtime_version_; }
  uint64_t code_object_hash() const { return code_hash_; }
  void *function(const std::string &symbol) const; // hipFunction_t
  void make_current() const;

private:
  Context() = default;
  int device_ = 0;
  uint32_t cu_count_ = 0;
  std::string name_, arch_;
  int runtime_version_ = 0;
  uint64_t code_hash_ = 0;
  std::vector<void *> modules_;
  std::vector<std::pair<std::string, void *>> functions_;
};

class Executor;
struct ExecutorImpl;

// src/executor/prepared.rs:46-353: validated + routed op batch recorded
// once as a hipGraph and replayed with one launch per call.
class PreparedOps {
public:
  ~PreparedOps();
  PreparedOps(const PreparedOps &) = delete;
  PreparedOps &operator=(const PreparedOps &) = delete;
  RunStats run();
  void run_silent();
  void submit();
  RunStats wait();
  size_t n_calls() const { return n_calls_; }

private:
  friend class Executor;
  friend struct ExecutorImpl;
  PreparedOps() = default;
  const Executor *exec_ = nullptr;
  void *stream_ = nullptr; // hipStream_t
  void *graph_exec_ = nullptr;
  void *ev_start_ = nullptr, *ev_end_ = nullptr;
  std::vector<void *> scratch_;
  void *mlp_scratch_ = nullptr; // decode-MLP region inside scratch_
  uint64_t mlp_bytes_ = 0;
  void *status_ = nullptr; // decode-MLP wait status word, when the graph has one
  bool in_flight_ = false;
  bool submitted_once_ = false;
  size_t n_calls_ = 0;
  uint64_t flops_ = 0;
};

struct ExecutorImpl;

// src/executor/mod.rs:102-391: thread-safe dispatcher over a pool of
// slots (a slot = one HIP stream + its events and scratch).
class Executor {
public:
  Executor(std::shared_ptr<Context> ctx, KernelSelection selection, ExecutorConfig config);
  // ML_TUNE read from the environment (src/executor/mod.rs:325-339).
  Executor(std::shared_ptr<Context> ctx, KernelSelection selection, size_t n_slots,
           uint32_t max_calls_per_submit);
  ~Executor();
  Executor(const Executor &) = delete;
  Executor &operator=(const Executor &) = delete;

  const std::shared_ptr<Context> &context() const;

  RunStats run_matmuls(const std::vector<MatmulCall> &calls) const;
  RunStats run_matmul_graph(const std::vector<MatmulCall> &calls) const;
  RunStats run_ops(const std::vector<MatmulOp> &ops) const;
  RunStats run_op_graph(const std::vector<MatmulOp> &ops) const;
  // src/executor/elementwise/gemv_chain.rs:14-194 (run_gemv_chain): up to
  // kGemvChainMaxJobs M = 1 row GEMVs on row-major f16 weights, validated
  // with the reference's rules, run in list order (each job sees the
  // earlier jobs' writes) on the decode GEMV launches.
  RunStats run_gemv_chain(const std::vector<MatmulOp> &jobs) const;
  RunStats run_matmuls_split_k2(const MatmulCall &call, uint32_t num_k_splits) const;
  // run_matmuls_split_k2 for a whole op: the reduce applies the op's
  // fused epilogue (accumulate, bias, activation, binary with D) once to
  // the fixed-order plane sum.  No reference counterpart: the reference
  // splits plain calls only (src/executor/mod.rs:179-210).
  RunStats run_op_split_k2(const MatmulOp &op, uint32_t num_k_splits) const;
  // run_matmuls_split_k2 without allocating: partial planes live in a
  // fixed per-device array of TA_NOALLOC_SCRATCH_BYTES (no reference
  // counterpart; for callers that cannot allocate device memory).
  RunStats run_matmuls_split_k2_noalloc(const MatmulCall &call, uint32_t num_k_splits) const;

  // Model ops (src/executor/elementwise/ops.rs); in-place (input ==
  // output) is allowed except for the copy.
  RunStats run_softmax_rows(const Tensor &input, const Tensor &output, float scale,
                            SoftmaxMask mask) const;
  RunStats run_rms_norm(const Tensor &input, const Tensor &weight, const Tensor &output,
                        float eps) const;
  RunStats run_layer_norm(const Tensor &input, const Tensor &weight, const Tensor &bias,
                          const Tensor &output, float eps) const;
  RunStats run_rope(const Tensor &input, const Tensor &table, const Tensor &output,
                    const RopeDesc &desc) const;
  RunStats run_copy_strided(const Tensor &src, const Tensor &dst, const CopyDesc &desc) const;
  // ops.rs:243-380 and flash.rs:255-402: RoPE scattered into a cache,
  // the binary combine, and the f16 prefill QKV pack.
  RunStats run_rope_scatter(const Tensor &input, const Tensor &table, const Tensor &dst,
                            const RopeDesc &desc, const RopeScatterDesc &scatter) const;
  RunStats run_binary(const Tensor &a, const Tensor &b, const Tensor &out, BinaryOp op) const;
  RunStats run_prefill_qkv_pack(const Tensor &qkv, const Tensor &table, const Tensor &q,
                                const Tensor &kt, const Tensor &v,
                                const PrefillQkvPackDesc &desc) const;
  // src/executor/elementwise/flash.rs:13-250: kt [H_kv, dh, T_max],
  // v [H_kv, T_max, dh], dh 64 or 128, H a multiple of H_kv.
  RunStats run_flash_attention(const Tensor &q, const Tensor &kt, const Tensor &v,
                               const Tensor &out, const FlashAttentionDesc &desc) const;
  // flash.rs:41-50: the reference's SIMT route.  There is one route here,
  // the same kernels as run_flash_attention.
  RunStats run_flash_attention_simt(const Tensor &q, const Tensor &kt, const Tensor &v,
                                    const Tensor &out, const FlashAttentionDesc &desc) const {
    return run_flash_attention(q, kt, v, out, desc);
  }
  // The GPU token loop (elementwise/ops.rs:456-595, attn.rs:14-185):
  // greedy argmax into a cell, the embedding rows of the cell's token ids
  // (out [embd] or [t, embd]), and split-K decode attention (q / out
  // [kv_heads, group, dh], group <= 8, dh 64 or 128).
  RunStats run_argmax(const Tensor &input, const U32Cell &result) const;
  RunStats run_embed_gather(const U32Cell &tokens, const Tensor &table, const Tensor &out) const;
  RunStats run_attn_decode(const Tensor &q, const Tensor &kt, const Tensor &v,
                           const Tensor &scratch, const Tensor &out,
                           const AttnDecodeDesc &desc) const;

  // Mixed-op graphs (src/executor/graph_ops.rs:244-336): every op is
  // validated and planned before anything is launched.
  RunStats run_exec_ops(const std::vector<ExecOp> &ops) const;
  std::unique_ptr<PreparedOps> prepare_exec_ops(const std::vector<ExecOp> &ops) const;

  std::unique_ptr<PreparedOps> prepare_matmuls(const std::vector<MatmulCall> &calls) const;
  std::unique_ptr<PreparedOps> prepare_ops(const std::vector<MatmulOp> &ops) const;
  std::unique_ptr<PreparedOps> prepare_op_graph(const std::vector<MatmulOp> &ops) const;

  void tune_shape(uint32_t batch, uint32_t m, uint32_t n, uint32_t k) const;
  DispatchInfo dispatch_info(uint32_t batch, uint32_t m, uint32_t n, uint32_t k) const;
  DispatchInfo dispatch_info_for(uint32_t batch, uint32_t m, uint32_t n, uint32_t k,
                                 bool b_f16) const;

  void upload(const float *src, size_t len, const Tensor &dst) const;
  void upload_f16(const uint16_t *src, size_t len, const Tensor &dst) const;
  void download(const Tensor &src, float *dst, size_t len) const;

  ExecutorImpl *impl() const { return impl_.get(); }

private:
  std::unique_ptr<ExecutorImpl> impl_;
};

} // namespace tensor_ash
