// The C ABI of include/tensor_ash.h over the C++ runtime.
// Conventions of the reference capi crate (capi/src/error.rs:8-121,
// capi/src/handles.rs): 0 / -1 / NULL returns, a thread-local error
// string cleared at every call, no exception crosses the boundary,
// destroying NULL is a no-op, "<fn>: <arg> is null" messages.
#include <cstring>
#include <functional>

#include "../../../include/tensor_ash.h"
#include "internal.hpp"

static_assert(TA_NOALLOC_SCRATCH_BYTES == TA_FIXED_SCRATCH_BYTES,
              "include/tensor_ash.h and kernel_args.h disagree on the fixed scratch size");

using namespace tensor_ash;

struct ta_context {
  std::shared_ptr<Context> ctx;
};
struct ta_executor {
  std::shared_ptr<Context> ctx;
  std::unique_ptr<Executor> exec;
};
struct ta_tensor {
  std::shared_ptr<Context> ctx;
  Tensor tensor;
};
struct ta_prepared {
  std::unique_ptr<PreparedOps> prepared;
  std::shared_ptr<Context> ctx;
};
struct ta_u32_cell {
  std::unique_ptr<U32Cell> cell;
};

namespace {

thread_local std::string g_last_error;

void set_error(const std::string &e) { g_last_error = e; }

int ffi_status(const std::function<void()> &f) {
  g_last_error.clear();
  try {
    f();
    return 0;
  } catch (const std::exception &e) {
    set_error(e.what());
  } catch (...) {
    set_error("panic crossed tensor-ash C ABI boundary");
  }
  return -1;
}

template <typename T> T *ffi_create(const std::function<T *()> &f) {
  g_last_error.clear();
  try {
    return f();
  } catch (const std::exception &e) {
    set_error(e.what());
  } catch (...) {
    set_error("panic crossed tensor-ash C ABI boundary");
  }
  return nullptr;
}

template <typename T> const T &checked_ref(const T *p, const std::string &msg) {
  if (!p)
    fail(msg);
  return *p;
}

std::string opt_str(const char *p, const char *dflt) { return p ? std::string(p) : dflt; }

const Tensor *checked_tensor(const ta_executor &e, const ta_tensor *t, const std::string &op,
                             const char *operand) {
  if (!t)
    fail(op + ": " + operand + " is null");
  if (t->ctx != e.ctx)
    fail(op + ": " + operand + " belongs to a different HIP context");
  return &t->tensor;
}

MatmulCall checked_call(const ta_executor &e, const ta_matmul_call &raw, const std::string &op) {
  MatmulCall c;
  c.a = checked_tensor(e, raw.a, op, "a");
  c.b = checked_tensor(e, raw.b, op, "b");
  c.c = checked_tensor(e, raw.c, op, "c");
  c.alpha = raw.alpha;
  c.accumulate = raw.accumulate != 0;
  return c;
}

// capi/src/api/ops.rs:15-71.
MatmulOp checked_op(const ta_executor &e, const ta_matmul_op &raw, const std::string &op) {
  MatmulOp o(checked_call(e, raw.call, op));
  const ta_epilogue &ep = raw.epilogue;
  if (ep.bias)
    o.epilogue.bias = checked_tensor(e, ep.bias, op, "epilogue.bias");
  if (ep.activation > 3)
    fail(op + ": epilogue.activation " + std::to_string(ep.activation) +
         " is invalid (0=none 1=relu 2=silu 3=gelu)");
  o.epilogue.activation = (Activation)ep.activation;
  switch (ep.binary_kind) {
  case 0:
    if (ep.d)
      fail(op + ": epilogue.d is set but binary_kind is 0 (none)");
    break;
  case 1:
    o.epilogue.binary = EpilogueBinary::add_scaled(*checked_tensor(e, ep.d, op, "epilogue.d"),
                                                   ep.beta);
    break;
  case 2:
    o.epilogue.binary = EpilogueBinary::mul(*checked_tensor(e, ep.d, op, "epilogue.d"));
    break;
  default:
    fail(op + ": epilogue.binary_kind " + std::to_string(ep.binary_kind) +
         " is invalid (0=none 1=add_scaled 2=mul)");
  }
  return o;
}

std::vector<MatmulOp> checked_ops(const ta_executor &e, const ta_matmul_op *ops, size_t n,
                                  const std::string &op) {
  if (n > 0 && !ops)
    fail(op + ": ops is null");
  std::vector<MatmulOp> out;
  for (size_t i = 0; i < n; ++i)
    out.push_back(checked_op(e, ops[i], op + ": op " + std::to_string(i)));
  return out;
}

std::vector<MatmulOp> checked_ops_v2(const ta_executor &e, const ta_matmul_op_v2 *ops, size_t n,
                                     const std::string &op) {
  if (n > 0 && !ops)
    fail(op + ": ops is null");
  std::vector<MatmulOp> out;
  for (size_t i = 0; i < n; ++i) {
    const std::string where = op + ": op " + std::to_string(i);
    if (ops[i].reserved[0] || ops[i].reserved[1] || ops[i].reserved[2])
      fail(where + ": reserved fields must be zero");
    MatmulOp o = checked_op(e, ops[i].base, where);
    o.packed_b = ops[i].packed_b != 0;
    out.push_back(o);
  }
  return out;
}

std::vector<MatmulOp> checked_ops_v3(const ta_executor &e, const ta_matmul_op_v3 *ops, size_t n,
                                     const std::string &op) {
  if (n > 0 && !ops)
    fail(op + ": ops is null");
  std::vector<MatmulOp> out;
  for (size_t i = 0; i < n; ++i) {
    const std::string where = op + ": op " + std::to_string(i);
    const ta_matmul_op_v3 &v = ops[i];
    std::vector<MatmulOp> base = checked_ops_v2(e, &v.v2, 1, where);
    MatmulOp o = base[0];
    if (v.norm_weight)
      o.normed_a = NormedA{checked_tensor(e, v.norm_weight, where, "norm_weight"), v.norm_eps};
    if (v.store.reserved)
      fail(where + ": store.reserved must be zero");
    MatmulStoreDesc d;
    d.head_dim = v.store.head_dim;
    d.pos_base = v.store.pos_base;
    d.pos_scale = v.store.pos_scale;
    d.stride_head = v.store.stride_head;
    d.stride_dim = v.store.stride_dim;
    d.pos_addr = v.store.pos_addr;
    switch (v.store_kind) {
    case TA_STORE_NONE:
      if (v.store_table || v.store_dst)
        fail(where + ": store tensors are set but store_kind is 0 (none)");
      break;
    case TA_STORE_ROPE:
      o = o.with_store_rope(*checked_tensor(e, v.store_table, where, "store_table"), d);
      break;
    case TA_STORE_SCATTER:
      o = o.with_store_scatter(*checked_tensor(e, v.store_dst, where, "store_dst"), d);
      break;
    case TA_STORE_ROPE_SCATTER:
      o = o.with_store_rope_scatter(*checked_tensor(e, v.store_table, where, "store_table"),
                                    *checked_tensor(e, v.store_dst, where, "store_dst"), d);
      break;
    default:
      fail(where + ": store_kind " + std::to_string(v.store_kind) +
           " is invalid (0=none 1=rope 2=scatter 3=rope_scatter)");
    }
    out.push_back(o);
  }
  return out;
}

// capi/src/api/matmul.rs:86-103.
void write_stats(ta_run_stats *out, const RunStats &s) {
  if (!out)
    return;
  out->has_gpu_time = s.gpu_time_ns ? 1 : 0;
  out->gpu_time_ns = s.gpu_time_ns.value_or(0);
  out->n_calls = s.n_calls;
  out->total_flops = s.total_flops;
  out->tflops = s.tflops().value_or(__builtin_nan(""));
}

std::vector<uint32_t> checked_shape(const uint32_t *shape, size_t rank, const std::string &op) {
  if (rank > 0 && !shape)
    fail(op + ": shape is null");
  return std::vector<uint32_t>(shape, shape + rank);
}

template <typename T> void destroy_handle(T *p) {
  if (!p)
    return;
  g_last_error.clear();
  try {
    delete p;
  } catch (...) {
    set_error("panic crossed tensor-ash C ABI boundary");
  }
}

} // namespace

extern "C" {

const char *ta_version(void) { return "2.0.0-gfx950"; }
const char *ta_last_error(void) { return g_last_error.c_str(); }

ta_context *ta_context_create(uint32_t enable_validation, const char *device_preference) {
  return ffi_create<ta_context>([&] {
    auto ctx = Context::create(enable_validation != 0, opt_str(device_preference, "auto"));
    return new ta_context{ctx};
  });
}

void ta_context_destroy(ta_context *ctx) { destroy_handle(ctx); }

uint32_t ta_context_supports_f16(const ta_context *ctx) { return ctx ? 1u : 0u; }
uint32_t ta_context_supports_bda(const ta_context *ctx) { return ctx ? 1u : 0u; }
uint32_t ta_context_cu_count(const ta_context *ctx) { return ctx ? ctx->ctx->cu_count() : 0u; }

static ta_executor *make_executor(const ta_context *ctx, size_t n_slots, uint32_t max_calls,
                                  const char *sel, std::optional<bool> tune, const char *fn) {
  return ffi_create<ta_executor>([&] {
    const ta_context &c = checked_ref(ctx, std::string(fn) + ": ctx is null");
    KernelSelection s = KernelSelection::parse(opt_str(sel, "auto"));
    std::unique_ptr<Executor> e;
    if (tune)
      e.reset(new Executor(c.ctx, s, ExecutorConfig{n_slots, max_calls, *tune}));
    else
      e.reset(new Executor(c.ctx, s, n_slots, max_calls));
    return new ta_executor{c.ctx, std::move(e)};
  });
}

ta_executor *ta_executor_create(const ta_context *ctx, size_t n_slots,
                                uint32_t max_calls_per_submit, const char *kernel_selection) {
  return make_executor(ctx, n_slots, max_calls_per_submit, kernel_selection, std::nullopt,
                       "ta_executor_create");
}

ta_executor *ta_executor_create_v2(const ta_context *ctx, size_t n_slots,
                                   uint32_t max_calls_per_submit, const char *kernel_selection,
                                   uint32_t tune) {
  return make_executor(ctx, n_slots, max_calls_per_submit, kernel_selection, tune != 0,
                       "ta_executor_create_v2");
}

void ta_executor_destroy(ta_executor *exec) { destroy_handle(exec); }

static ta_tensor *make_tensor(const std::shared_ptr<Context> &ctx, const uint32_t *shape,
                              size_t rank, bool f16, const std::string &fn) {
  auto s = checked_shape(shape, rank, fn);
  Tensor t = f16 ? Tensor::uninit_device_f16(ctx, s) : Tensor::uninit_device(ctx, s);
  return new ta_tensor{ctx, t};
}

ta_tensor *ta_tensor_create(const ta_context *ctx, const uint32_t *shape, size_t rank) {
  return ffi_create<ta_tensor>([&] {
    const ta_context &c = checked_ref(ctx, "ta_tensor_create: ctx is null");
    return make_tensor(c.ctx, shape, rank, false, "ta_tensor_create");
  });
}
ta_tensor *ta_tensor_create_on_executor(const ta_executor *exec, const uint32_t *shape,
                                        size_t rank) {
  return ffi_create<ta_tensor>([&] {
    const ta_executor &e = checked_ref(exec, "ta_tensor_create_on_executor: exec is null");
    return make_tensor(e.ctx, shape, rank, false, "ta_tensor_create_on_executor");
  });
}
ta_tensor *ta_tensor_create_f16(const ta_context *ctx, const uint32_t *shape, size_t rank) {
  return ffi_create<ta_tensor>([&] {
    const ta_context &c = checked_ref(ctx, "ta_tensor_create_f16: ctx is null");
    return make_tensor(c.ctx, shape, rank, true, "ta_tensor_create_f16");
  });
}
ta_tensor *ta_tensor_create_f16_on_executor(const ta_executor *exec, const uint32_t *shape,
                                            size_t rank) {
  return ffi_create<ta_tensor>([&] {
    const ta_executor &e = checked_ref(exec, "ta_tensor_create_f16_on_executor: exec is null");
    return make_tensor(e.ctx, shape, rank, true, "ta_tensor_create_f16_on_executor");
  });
}

void ta_tensor_destroy(ta_tensor *t) { destroy_handle(t); }
uint64_t ta_tensor_len(const ta_tensor *t) { return t ? t->tensor.len() : 0; }
uint64_t ta_tensor_size_bytes(const ta_tensor *t) { return t ? t->tensor.size_bytes() : 0; }
uint32_t ta_tensor_is_f16(const ta_tensor *t) {
  return t && t->tensor.dtype() == DType::F16 ? 1u : 0u;
}
uint64_t ta_tensor_device_address(const ta_tensor *t) {
  return t ? (uint64_t)(uintptr_t)t->tensor.device_ptr() : 0;
}

int ta_upload(const ta_executor *exec, const ta_tensor *dst, const float *src, size_t len) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_upload: exec is null");
    const Tensor *t = checked_tensor(e, dst, "ta_upload", "dst");
    if (len > 0 && !src)
      fail("ta_upload: src is null");
    e.exec->upload(src, len, *t);
  });
}

int ta_upload_f16(const ta_executor *exec, const ta_tensor *dst, const uint16_t *src, size_t len) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_upload_f16: exec is null");
    const Tensor *t = checked_tensor(e, dst, "ta_upload_f16", "dst");
    if (len > 0 && !src)
      fail("ta_upload_f16: src is null");
    e.exec->upload_f16(src, len, *t);
  });
}

int ta_download(const ta_executor *exec, const ta_tensor *src, float *dst, size_t len) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_download: exec is null");
    const Tensor *t = checked_tensor(e, src, "ta_download", "src");
    if (len > 0 && !dst)
      fail("ta_download: dst is null");
    e.exec->download(*t, dst, len);
  });
}

int ta_matmul(const ta_executor *exec, const ta_tensor *a, const ta_tensor *b,
              const ta_tensor *c, float alpha, uint32_t accumulate, ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_matmul: exec is null");
    ta_matmul_call raw{a, b, c, alpha, accumulate};
    write_stats(stats, e.exec->run_matmuls({checked_call(e, raw, "ta_matmul")}));
  });
}

int ta_matmul_batch(const ta_executor *exec, const ta_matmul_call *calls, size_t n_calls,
                    ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_matmul_batch: exec is null");
    if (n_calls > 0 && !calls)
      fail("ta_matmul_batch: calls is null");
    std::vector<MatmulCall> cs;
    for (size_t i = 0; i < n_calls; ++i)
      cs.push_back(checked_call(e, calls[i], "ta_matmul_batch: call " + std::to_string(i)));
    write_stats(stats, e.exec->run_matmuls(cs));
  });
}

int ta_run_ops(const ta_executor *exec, const ta_matmul_op *ops, size_t n_ops,
               ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_run_ops: exec is null");
    write_stats(stats, e.exec->run_ops(checked_ops(e, ops, n_ops, "ta_run_ops")));
  });
}

int ta_run_op_graph(const ta_executor *exec, const ta_matmul_op *ops, size_t n_ops,
                    ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_run_op_graph: exec is null");
    write_stats(stats, e.exec->run_op_graph(checked_ops(e, ops, n_ops, "ta_run_op_graph")));
  });
}

int ta_run_ops_v2(const ta_executor *exec, const ta_matmul_op_v2 *ops, size_t n_ops,
                  ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_run_ops_v2: exec is null");
    write_stats(stats, e.exec->run_ops(checked_ops_v2(e, ops, n_ops, "ta_run_ops_v2")));
  });
}

int ta_run_ops_v3(const ta_executor *exec, const ta_matmul_op_v3 *ops, size_t n_ops,
                  ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_run_ops_v3: exec is null");
    write_stats(stats, e.exec->run_ops(checked_ops_v3(e, ops, n_ops, "ta_run_ops_v3")));
  });
}

int ta_run_op_graph_v3(const ta_executor *exec, const ta_matmul_op_v3 *ops, size_t n_ops,
                       ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_run_op_graph_v3: exec is null");
    write_stats(stats,
                e.exec->run_op_graph(checked_ops_v3(e, ops, n_ops, "ta_run_op_graph_v3")));
  });
}

int ta_run_gemv_chain(const ta_executor *exec, const ta_matmul_op_v3 *jobs, size_t n_jobs,
                      ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_run_gemv_chain: exec is null");
    write_stats(stats,
                e.exec->run_gemv_chain(checked_ops_v3(e, jobs, n_jobs, "ta_run_gemv_chain")));
  });
}

int ta_run_op_graph_v2(const ta_executor *exec, const ta_matmul_op_v2 *ops, size_t n_ops,
                       ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_run_op_graph_v2: exec is null");
    write_stats(stats,
                e.exec->run_op_graph(checked_ops_v2(e, ops, n_ops, "ta_run_op_graph_v2")));
  });
}

int ta_matmul_split_k2(const ta_executor *exec, const ta_tensor *a, const ta_tensor *b,
                       const ta_tensor *c, float alpha, uint32_t splits, ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_matmul_split_k2: exec is null");
    ta_matmul_call raw{a, b, c, alpha, 0};
    write_stats(stats,
                e.exec->run_matmuls_split_k2(checked_call(e, raw, "ta_matmul_split_k2"), splits));
  });
}

uint64_t ta_allocation_count(void) { return allocation_count(); }

int ta_run_op_split_k2(const ta_executor *exec, const ta_matmul_op *op, uint32_t splits,
                       ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_run_op_split_k2: exec is null");
    if (!op)
      fail("ta_run_op_split_k2: op is null");
    write_stats(stats,
                e.exec->run_op_split_k2(checked_op(e, *op, "ta_run_op_split_k2"), splits));
  });
}

int ta_matmul_split_k2_noalloc(const ta_executor *exec, const ta_tensor *a, const ta_tensor *b,
                               const ta_tensor *c, float alpha, uint32_t splits,
                               ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_matmul_split_k2_noalloc: exec is null");
    ta_matmul_call raw{a, b, c, alpha, 0};
    write_stats(stats, e.exec->run_matmuls_split_k2_noalloc(
                           checked_call(e, raw, "ta_matmul_split_k2_noalloc"), splits));
  });
}

namespace {
FlashAttentionDesc flash_desc(const ta_flash_desc &d, const std::string &fn) {
  if (d.reserved)
    fail(fn + ": flash.reserved must be zero");
  FlashAttentionDesc f;
  f.kv_len = d.kv_len;
  f.pos_base = d.pos_base;
  f.scale = d.scale;
  if (d.token_major_heads)
    f.token_major_heads = d.token_major_heads;
  if (d.out_token_major_heads)
    f.out_token_major_heads = d.out_token_major_heads;
  return f;
}
SoftmaxMask softmax_mask(uint32_t kind, uint32_t valid_or_prefix, uint32_t rows_per_group,
                         const std::string &fn) {
  switch (kind) {
  case TA_SOFTMAX_MASK_FULL:
    return SoftmaxMask::full();
  case TA_SOFTMAX_MASK_PREFIX:
    return SoftmaxMask::prefix_of(valid_or_prefix);
  case TA_SOFTMAX_MASK_CAUSAL:
    return SoftmaxMask::causal(valid_or_prefix, rows_per_group);
  default:
    fail(fn + ": mask_kind " + std::to_string(kind) + " is invalid (0=full 1=prefix 2=causal)");
  }
}
CopyDesc copy_desc(const ta_copy_desc &d) {
  CopyDesc cd;
  for (int i = 0; i < 3; ++i) {
    cd.extent[i] = d.extent[i];
    cd.src_strides[i] = d.src_strides[i];
    cd.dst_strides[i] = d.dst_strides[i];
  }
  cd.src_offset = d.src_offset;
  cd.dst_offset = d.dst_offset;
  return cd;
}
RopeDesc rope_desc(const ta_rope_desc &d) {
  RopeDesc rd;
  rd.heads = d.heads;
  rd.head_dim = d.head_dim;
  rd.rot_dim = d.rot_dim;
  rd.pos_base = d.pos_base;
  return rd;
}

const U32Cell *checked_cell(const ta_executor &e, const ta_u32_cell *c, const std::string &op,
                            const char *operand) {
  if (!c)
    fail(op + ": " + operand + " is null");
  if (c->cell->context() != e.ctx.get())
    fail(op + ": " + operand + " belongs to a different HIP context");
  return c->cell.get();
}

RopeScatterDesc scatter_desc(const ta_rope_scatter_desc &d, const std::string &fn) {
  if (d.reserved != 0)
    fail(fn + ": ta_rope_scatter_desc.reserved must be zero");
  RopeScatterDesc r;
  r.dst_offset = d.dst_offset;
  for (int i = 0; i < 3; ++i)
    r.dst_strides[i] = d.dst_strides[i];
  r.pos_scale = d.pos_scale;
  return r;
}

BinaryOp binary_op(uint32_t op, float beta, const std::string &fn) {
  if (op == TA_BINARY_OP_ADD_SCALED)
    return BinaryOp::add_scaled(beta);
  if (op == TA_BINARY_OP_SILU_MUL)
    return BinaryOp::silu_mul();
  fail(fn + ": binary op " + std::to_string(op) + " is invalid");
}

PrefillQkvPackDesc qkv_pack_desc(const ta_prefill_qkv_pack_desc &d, const std::string &fn) {
  if (d.reserved != 0)
    fail(fn + ": ta_prefill_qkv_pack_desc.reserved must be zero");
  PrefillQkvPackDesc r;
  r.heads = d.heads;
  r.kv_heads = d.kv_heads;
  r.head_dim = d.head_dim;
  r.rot_dim = d.rot_dim;
  r.pos_base = d.pos_base;
  return r;
}

AttnDecodeDesc attn_decode_desc(const ta_attn_decode_desc &d) {
  AttnDecodeDesc a;
  a.kv_len = d.kv_len;
  a.scale = d.scale;
  a.pos_addr = d.pos_addr;
  return a;
}

std::vector<ExecOp> checked_exec_ops(const ta_executor &e, const ta_exec_op *ops, size_t n,
                                     const std::string &fn) {
  if (n > 0 && !ops)
    fail(fn + ": ops is null");
  std::vector<ExecOp> out;
  for (size_t i = 0; i < n; ++i) {
    const std::string where = fn + ": op " + std::to_string(i);
    const ta_exec_op &o = ops[i];
    auto t = [&](const ta_tensor *x, const char *role) -> const Tensor & {
      return *checked_tensor(e, x, where, role);
    };
    switch (o.kind) {
    case TA_EXEC_MATMUL:
      if (!o.matmul)
        fail(where + ": matmul is null");
      out.push_back(ExecOp::from_matmul(checked_ops_v3(e, o.matmul, 1, where)[0]));
      break;
    case TA_EXEC_RMS_NORM:
      out.push_back(ExecOp::rms_norm(t(o.in[0], "input"), t(o.in[1], "weight"),
                                     t(o.out, "output"), o.scalar));
      break;
    case TA_EXEC_LAYER_NORM:
      out.push_back(ExecOp::layer_norm(t(o.in[0], "input"), t(o.in[1], "weight"),
                                       t(o.in[2], "bias"), t(o.out, "output"), o.scalar));
      break;
    case TA_EXEC_SOFTMAX_ROWS:
      out.push_back(ExecOp::softmax_rows(
          t(o.in[0], "input"), t(o.out, "output"), o.scalar,
          softmax_mask(o.mask_kind, o.valid_or_prefix, o.rows_per_group, where)));
      break;
    case TA_EXEC_ROPE: {
      RopeDesc rd = rope_desc(o.rope);
      rd.pos_addr = o.pos_addr;
      out.push_back(ExecOp::rope_op(t(o.in[0], "input"), t(o.in[1], "table"), t(o.out, "output"),
                                    rd));
      break;
    }
    case TA_EXEC_COPY_STRIDED: {
      CopyDesc cd = copy_desc(o.copy);
      cd.pos_addr = o.pos_addr;
      cd.pos_scale = o.pos_scale;
      out.push_back(ExecOp::copy_strided(t(o.in[0], "src"), t(o.out, "dst"), cd));
      break;
    }
    case TA_EXEC_FLASH_ATTENTION:
      out.push_back(ExecOp::flash_attn(t(o.in[0], "q"), t(o.in[1], "kt"), t(o.in[2], "v"),
                                       t(o.out, "out"), flash_desc(o.flash, where)));
      break;
    case TA_EXEC_ARGMAX:
      out.push_back(ExecOp::argmax(t(o.in[0], "input"), *checked_cell(e, o.cell, where, "cell")));
      break;
    case TA_EXEC_EMBED_GATHER:
      out.push_back(ExecOp::embed_gather(*checked_cell(e, o.cell, where, "cell"),
                                         t(o.in[0], "table"), t(o.out, "out")));
      break;
    case TA_EXEC_GEMV_CHAIN:
      if (!o.matmul && o.n_jobs > 0)
        fail(where + ": matmul is null");
      out.push_back(ExecOp::gemv_chain(checked_ops_v3(e, o.matmul, o.n_jobs, where)));
      break;
    case TA_EXEC_ROPE_SCATTER: {
      RopeDesc rd = rope_desc(o.rope);
      rd.pos_addr = o.pos_addr;
      out.push_back(ExecOp::rope_scatter(t(o.in[0], "input"), t(o.in[1], "table"), t(o.out, "dst"),
                                         rd, scatter_desc(o.scatter, where)));
      break;
    }
    case TA_EXEC_BINARY:
      out.push_back(ExecOp::binary_op(t(o.in[0], "a"), t(o.in[1], "b"), t(o.out, "out"),
                                      binary_op(o.binary_op, o.scalar, where)));
      break;
    case TA_EXEC_PREFILL_QKV_PACK:
      out.push_back(ExecOp::prefill_qkv_pack(t(o.in[0], "qkv"), t(o.in[1], "table"), t(o.out, "q"),
                                             t(o.aux, "kt"), t(o.aux2, "v"),
                                             qkv_pack_desc(o.qkv, where)));
      break;
    case TA_EXEC_ATTN_DECODE:
      out.push_back(ExecOp::attn_decode(t(o.in[0], "q"), t(o.in[1], "kt"), t(o.in[2], "v"),
                                        t(o.aux, "scratch"), t(o.out, "out"),
                                        attn_decode_desc(o.attn)));
      break;
    default:
      fail(where + ": kind " + std::to_string(o.kind) + " is invalid");
    }
  }
  return out;
}
} // namespace

// capi/src/api/elementwise.rs: the model ops.
int ta_softmax_rows(const ta_executor *exec, const ta_tensor *input, const ta_tensor *output,
                    float scale, uint32_t mask_kind, uint32_t valid_or_prefix,
                    uint32_t rows_per_group, ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_softmax_rows: exec is null");
    const Tensor *in = checked_tensor(e, input, "ta_softmax_rows", "input");
    const Tensor *out = checked_tensor(e, output, "ta_softmax_rows", "output");
    const SoftmaxMask mask =
        softmax_mask(mask_kind, valid_or_prefix, rows_per_group, "ta_softmax_rows");
    write_stats(stats, e.exec->run_softmax_rows(*in, *out, scale, mask));
  });
}

int ta_rms_norm(const ta_executor *exec, const ta_tensor *input, const ta_tensor *weight,
                const ta_tensor *output, float eps, ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_rms_norm: exec is null");
    const Tensor *in = checked_tensor(e, input, "ta_rms_norm", "input");
    const Tensor *w = checked_tensor(e, weight, "ta_rms_norm", "weight");
    const Tensor *out = checked_tensor(e, output, "ta_rms_norm", "output");
    write_stats(stats, e.exec->run_rms_norm(*in, *w, *out, eps));
  });
}

int ta_layer_norm(const ta_executor *exec, const ta_tensor *input, const ta_tensor *weight,
                  const ta_tensor *bias, const ta_tensor *output, float eps, ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_layer_norm: exec is null");
    const Tensor *in = checked_tensor(e, input, "ta_layer_norm", "input");
    const Tensor *w = checked_tensor(e, weight, "ta_layer_norm", "weight");
    const Tensor *b = checked_tensor(e, bias, "ta_layer_norm", "bias");
    const Tensor *out = checked_tensor(e, output, "ta_layer_norm", "output");
    write_stats(stats, e.exec->run_layer_norm(*in, *w, *b, *out, eps));
  });
}

int ta_rope(const ta_executor *exec, const ta_tensor *input, const ta_tensor *table,
            const ta_tensor *output, const ta_rope_desc *desc, ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_rope: exec is null");
    const Tensor *in = checked_tensor(e, input, "ta_rope", "input");
    const Tensor *t = checked_tensor(e, table, "ta_rope", "table");
    const Tensor *out = checked_tensor(e, output, "ta_rope", "output");
    const ta_rope_desc &d = checked_ref(desc, "ta_rope: desc is null");
    RopeDesc rd;
    rd.heads = d.heads;
    rd.head_dim = d.head_dim;
    rd.rot_dim = d.rot_dim;
    rd.pos_base = d.pos_base;
    write_stats(stats, e.exec->run_rope(*in, *t, *out, rd));
  });
}

int ta_copy_strided(const ta_executor *exec, const ta_tensor *src, const ta_tensor *dst,
                    const ta_copy_desc *desc, ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_copy_strided: exec is null");
    const Tensor *s_ = checked_tensor(e, src, "ta_copy_strided", "src");
    const Tensor *d_ = checked_tensor(e, dst, "ta_copy_strided", "dst");
    const ta_copy_desc &d = checked_ref(desc, "ta_copy_strided: desc is null");
    CopyDesc cd;
    for (int i = 0; i < 3; ++i) {
      cd.extent[i] = d.extent[i];
      cd.src_strides[i] = d.src_strides[i];
      cd.dst_strides[i] = d.dst_strides[i];
    }
    cd.src_offset = d.src_offset;
    cd.dst_offset = d.dst_offset;
    write_stats(stats, e.exec->run_copy_strided(*s_, *d_, cd));
  });
}


int ta_flash_attention(const ta_executor *exec, const ta_tensor *q, const ta_tensor *kt,
                       const ta_tensor *v, const ta_tensor *out, const ta_flash_desc *desc,
                       ta_run_stats *stats) {
  return ffi_status([&] {
    const char *fn = "ta_flash_attention";
    const ta_executor &e = checked_ref(exec, "ta_flash_attention: exec is null");
    const Tensor *tq = checked_tensor(e, q, fn, "q");
    const Tensor *tk = checked_tensor(e, kt, fn, "kt");
    const Tensor *tv = checked_tensor(e, v, fn, "v");
    const Tensor *to = checked_tensor(e, out, fn, "out");
    const ta_flash_desc &d = checked_ref(desc, "ta_flash_attention: desc is null");
    write_stats(stats, e.exec->run_flash_attention(*tq, *tk, *tv, *to, flash_desc(d, fn)));
  });
}

// src/executor/cells.rs:163-205.
ta_u32_cell *ta_u32_cell_create(ta_context *ctx, uint32_t cap) {
  return ffi_create<ta_u32_cell>([&] {
    const ta_context &c = checked_ref(ctx, "ta_u32_cell_create: ctx is null");
    return new ta_u32_cell{U32Cell::create(c.ctx, cap)};
  });
}
void ta_u32_cell_destroy(ta_u32_cell *cell) { delete cell; }
int ta_u32_cell_write(ta_u32_cell *cell, const uint32_t *values, size_t n) {
  return ffi_status([&] {
    ta_u32_cell &c = const_cast<ta_u32_cell &>(checked_ref(cell, "ta_u32_cell_write: cell is null"));
    if (n > 0 && !values)
      fail("ta_u32_cell_write: values is null");
    c.cell->write(values, n);
  });
}
int ta_u32_cell_read(const ta_u32_cell *cell, uint32_t *value) {
  return ffi_status([&] {
    const ta_u32_cell &c = checked_ref(cell, "ta_u32_cell_read: cell is null");
    if (!value)
      fail("ta_u32_cell_read: value is null");
    *value = c.cell->read();
  });
}
uint64_t ta_u32_cell_device_address(const ta_u32_cell *cell) {
  return cell ? cell->cell->device_address() : 0;
}
uint32_t ta_u32_cell_cap(const ta_u32_cell *cell) { return cell ? cell->cell->cap() : 0; }

// src/executor/elementwise/ops.rs:243-380 and flash.rs:255-402.
int ta_rope_scatter(const ta_executor *exec, const ta_tensor *input, const ta_tensor *table,
                    const ta_tensor *dst, const ta_rope_desc *desc,
                    const ta_rope_scatter_desc *scatter, ta_run_stats *stats) {
  return ffi_status([&] {
    const char *fn = "ta_rope_scatter";
    const ta_executor &e = checked_ref(exec, "ta_rope_scatter: exec is null");
    const Tensor *ti = checked_tensor(e, input, fn, "input");
    const Tensor *tt = checked_tensor(e, table, fn, "table");
    const Tensor *td = checked_tensor(e, dst, fn, "dst");
    const ta_rope_desc &d = checked_ref(desc, "ta_rope_scatter: desc is null");
    const ta_rope_scatter_desc &sd = checked_ref(scatter, "ta_rope_scatter: scatter is null");
    write_stats(stats, e.exec->run_rope_scatter(*ti, *tt, *td, rope_desc(d), scatter_desc(sd, fn)));
  });
}
int ta_binary(const ta_executor *exec, const ta_tensor *a, const ta_tensor *b,
              const ta_tensor *out, uint32_t op, float beta, ta_run_stats *stats) {
  return ffi_status([&] {
    const char *fn = "ta_binary";
    const ta_executor &e = checked_ref(exec, "ta_binary: exec is null");
    const Tensor *ta_ = checked_tensor(e, a, fn, "a");
    const Tensor *tb = checked_tensor(e, b, fn, "b");
    const Tensor *to = checked_tensor(e, out, fn, "out");
    write_stats(stats, e.exec->run_binary(*ta_, *tb, *to, binary_op(op, beta, fn)));
  });
}
int ta_prefill_qkv_pack(const ta_executor *exec, const ta_tensor *qkv, const ta_tensor *table,
                        const ta_tensor *q, const ta_tensor *kt, const ta_tensor *v,
                        const ta_prefill_qkv_pack_desc *desc, ta_run_stats *stats) {
  return ffi_status([&] {
    const char *fn = "ta_prefill_qkv_pack";
    const ta_executor &e = checked_ref(exec, "ta_prefill_qkv_pack: exec is null");
    const Tensor *tx = checked_tensor(e, qkv, fn, "qkv");
    const Tensor *tt = checked_tensor(e, table, fn, "table");
    const Tensor *tq = checked_tensor(e, q, fn, "q");
    const Tensor *tk = checked_tensor(e, kt, fn, "kt");
    const Tensor *tv = checked_tensor(e, v, fn, "v");
    const ta_prefill_qkv_pack_desc &d = checked_ref(desc, "ta_prefill_qkv_pack: desc is null");
    write_stats(stats, e.exec->run_prefill_qkv_pack(*tx, *tt, *tq, *tk, *tv, qkv_pack_desc(d, fn)));
  });
}

// src/executor/elementwise/ops.rs:456-595 and attn.rs:14-185.
int ta_argmax(const ta_executor *exec, const ta_tensor *input, ta_u32_cell *result,
              ta_run_stats *stats) {
  return ffi_status([&] {
    const char *fn = "ta_argmax";
    const ta_executor &e = checked_ref(exec, "ta_argmax: exec is null");
    const Tensor *in = checked_tensor(e, input, fn, "input");
    write_stats(stats, e.exec->run_argmax(*in, *checked_cell(e, result, fn, "result")));
  });
}
int ta_embed_gather(const ta_executor *exec, const ta_u32_cell *tokens, const ta_tensor *table,
                    const ta_tensor *out, ta_run_stats *stats) {
  return ffi_status([&] {
    const char *fn = "ta_embed_gather";
    const ta_executor &e = checked_ref(exec, "ta_embed_gather: exec is null");
    const U32Cell *tc = checked_cell(e, tokens, fn, "tokens");
    const Tensor *tt = checked_tensor(e, table, fn, "table");
    const Tensor *to = checked_tensor(e, out, fn, "out");
    write_stats(stats, e.exec->run_embed_gather(*tc, *tt, *to));
  });
}
int ta_attn_decode(const ta_executor *exec, const ta_tensor *q, const ta_tensor *kt,
                   const ta_tensor *v, const ta_tensor *scratch, const ta_tensor *out,
                   const ta_attn_decode_desc *desc, ta_run_stats *stats) {
  return ffi_status([&] {
    const char *fn = "ta_attn_decode";
    const ta_executor &e = checked_ref(exec, "ta_attn_decode: exec is null");
    const Tensor *tq = checked_tensor(e, q, fn, "q");
    const Tensor *tk = checked_tensor(e, kt, fn, "kt");
    const Tensor *tv = checked_tensor(e, v, fn, "v");
    const Tensor *ts = checked_tensor(e, scratch, fn, "scratch");
    const Tensor *to = checked_tensor(e, out, fn, "out");
    const ta_attn_decode_desc &d = checked_ref(desc, "ta_attn_decode: desc is null");
    write_stats(stats, e.exec->run_attn_decode(*tq, *tk, *tv, *ts, *to, attn_decode_desc(d)));
  });
}

int ta_run_exec_ops(const ta_executor *exec, const ta_exec_op *ops, size_t n_ops,
                    ta_run_stats *stats) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_run_exec_ops: exec is null");
    write_stats(stats, e.exec->run_exec_ops(checked_exec_ops(e, ops, n_ops, "ta_run_exec_ops")));
  });
}

ta_prepared *ta_prepared_create_exec(const ta_executor *exec, const ta_exec_op *ops,
                                     size_t n_ops) {
  return ffi_create<ta_prepared>([&] {
    const ta_executor &e = checked_ref(exec, "ta_prepared_create_exec: exec is null");
    auto p = e.exec->prepare_exec_ops(checked_exec_ops(e, ops, n_ops, "ta_prepared_create_exec"));
    return new ta_prepared{std::move(p), e.ctx};
  });
}

static ta_prepared *make_prepared(const ta_executor *exec, std::vector<MatmulOp> (*conv)(
                                                                const ta_executor &, const void *,
                                                                size_t, const std::string &),
                                  const void *ops, size_t n_ops, uint32_t as_graph,
                                  const char *fn) {
  return ffi_create<ta_prepared>([&] {
    const ta_executor &e = checked_ref(exec, std::string(fn) + ": exec is null");
    auto v = conv(e, ops, n_ops, fn);
    auto p = as_graph ? e.exec->prepare_op_graph(v) : e.exec->prepare_ops(v);
    return new ta_prepared{std::move(p), e.ctx};
  });
}

ta_prepared *ta_prepared_create(const ta_executor *exec, const ta_matmul_op *ops, size_t n_ops,
                                uint32_t as_graph) {
  return make_prepared(
      exec,
      [](const ta_executor &e, const void *o, size_t n, const std::string &fn) {
        return checked_ops(e, static_cast<const ta_matmul_op *>(o), n, fn);
      },
      ops, n_ops, as_graph, "ta_prepared_create");
}

ta_prepared *ta_prepared_create_v2(const ta_executor *exec, const ta_matmul_op_v2 *ops,
                                   size_t n_ops, uint32_t as_graph) {
  return make_prepared(
      exec,
      [](const ta_executor &e, const void *o, size_t n, const std::string &fn) {
        return checked_ops_v2(e, static_cast<const ta_matmul_op_v2 *>(o), n, fn);
      },
      ops, n_ops, as_graph, "ta_prepared_create_v2");
}

ta_prepared *ta_prepared_create_v3(const ta_executor *exec, const ta_matmul_op_v3 *ops,
                                   size_t n_ops, uint32_t as_graph) {
  return make_prepared(
      exec,
      [](const ta_executor &e, const void *o, size_t n, const std::string &fn) {
        return checked_ops_v3(e, static_cast<const ta_matmul_op_v3 *>(o), n, fn);
      },
      ops, n_ops, as_graph, "ta_prepared_create_v3");
}

int ta_prepared_run(ta_prepared *prepared, ta_run_stats *stats) {
  return ffi_status([&] {
    if (!prepared)
      fail("ta_prepared_run: prepared is null");
    write_stats(stats, prepared->prepared->run());
  });
}
int ta_prepared_submit(ta_prepared *prepared) {
  return ffi_status([&] {
    if (!prepared)
      fail("ta_prepared_submit: prepared is null");
    prepared->prepared->submit();
  });
}
int ta_prepared_wait(ta_prepared *prepared, ta_run_stats *stats) {
  return ffi_status([&] {
    if (!prepared)
      fail("ta_prepared_wait: prepared is null");
    write_stats(stats, prepared->prepared->wait());
  });
}
void ta_prepared_destroy(ta_prepared *prepared) { destroy_handle(prepared); }

int ta_dispatch_info_for(const ta_executor *exec, uint32_t batch, uint32_t m, uint32_t n,
                         uint32_t k, uint32_t b_f16, ta_dispatch_info *out) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_dispatch_info_for: exec is null");
    if (!out)
      fail("ta_dispatch_info_for: out is null");
    DispatchInfo info = e.exec->dispatch_info_for(batch, m, n, k, b_f16 != 0);
    out->kernel = info.kernel; // registry names are static strings
    out->tile[0] = info.tile[0];
    out->tile[1] = info.tile[1];
    out->tile[2] = info.tile[2];
    out->has_split_k2 = info.split_k2_splits ? 1u : 0u;
    out->split_k2_splits = info.split_k2_splits.value_or(0);
  });
}

int ta_tune_shape(const ta_executor *exec, uint32_t batch, uint32_t m, uint32_t n, uint32_t k) {
  return ffi_status([&] {
    const ta_executor &e = checked_ref(exec, "ta_tune_shape: exec is null");
    e.exec->tune_shape(batch, m, n, k);
  });
}

int ta_pack_f16w_row_tiles(const float *src, size_t k, size_t n, size_t tile_n, float *dst) {
  return ffi_status([&] {
    if (k * n > 0 && (!src || !dst))
      fail("ta_pack_f16w_row_tiles: src or dst is null");
    auto v = pack_f16w_row_tiles(src, k, n, tile_n);
    if (!v.empty())
      std::memcpy(dst, v.data(), v.size() * sizeof(float));
  });
}

uint32_t ta_f16w_row_tile_n(uint32_t k, uint32_t n) { return f16w_row_tile_n(k, n); }

size_t ta_kernel_count(void) { return KERNEL_SPECS_LEN; }
const char *ta_kernel_name(size_t i) { return i < KERNEL_SPECS_LEN ? KERNEL_SPECS[i].name : nullptr; }
int ta_kernel_tile(size_t i, uint32_t *tile) {
  if (i >= KERNEL_SPECS_LEN || !tile)
    return -1;
  tile[0] = KERNEL_SPECS[i].tile_m;
  tile[1] = KERNEL_SPECS[i].tile_n;
  tile[2] = KERNEL_SPECS[i].tile_k;
  return 0;
}

} // extern "C"
