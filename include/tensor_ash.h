/*
 * tensor-ash C ABI, MI355X (gfx950) implementation.
 *
 * Drop-in for the reference's C header (gusahlg/tensor-ash
 * include/tensor_ash.h:1-244): same symbol names, argument order, struct
 * layouts, 0 / -1 / NULL return convention and thread-local
 * ta_last_error().  Every declaration below cites the reference line it
 * replaces; the additive extensions at the end have no reference C
 * counterpart (they expose Rust-API features the reference's C ABI leaves
 * out, capi/src/api/ops.rs:65-69) and never change an existing layout.
 */
#ifndef TENSOR_ASH_H
#define TENSOR_ASH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ta_context ta_context;   /* ref tensor_ash.h:11 */
typedef struct ta_executor ta_executor; /* ref tensor_ash.h:12 */
typedef struct ta_tensor ta_tensor;     /* ref tensor_ash.h:13 */
typedef struct ta_prepared ta_prepared; /* ref tensor_ash.h:14 */

/* ref tensor_ash.h:16-22.  gpu_time_ns is measured with hipEvents around
 * the submission on its stream. */
typedef struct ta_run_stats {
  uint32_t has_gpu_time;
  uint64_t gpu_time_ns;
  size_t n_calls;
  uint64_t total_flops;
  double tflops;
} ta_run_stats;

/* ref tensor_ash.h:24-30.  C <- alpha * A @ B (+ C if accumulate). */
typedef struct ta_matmul_call {
  const ta_tensor *a;
  const ta_tensor *b;
  const ta_tensor *c;
  float alpha;
  uint32_t accumulate;
} ta_matmul_call;

/* ref tensor_ash.h:33-38. */
enum {
  TA_ACTIVATION_NONE = 0,
  TA_ACTIVATION_RELU = 1,
  TA_ACTIVATION_SILU = 2, /* x * sigmoid(x) */
  TA_ACTIVATION_GELU = 3  /* tanh-approximated GELU */
};

/* ref tensor_ash.h:41-45. */
enum {
  TA_BINARY_NONE = 0,
  TA_BINARY_ADD_SCALED = 1, /* out = act_result + beta * D */
  TA_BINARY_MUL = 2         /* out = act_result * D */
};

/* ref tensor_ash.h:47-59.  Applied while the output tile is in
 * registers: +bias -> activation -> binary op with D.  bias is [N] or
 * [B, N]; d must be non-null iff binary_kind != 0 and has C's shape. */
typedef struct ta_epilogue {
  const ta_tensor *bias;
  uint32_t activation;  /* TA_ACTIVATION_* */
  uint32_t binary_kind; /* TA_BINARY_* */
  const ta_tensor *d;
  float beta; /* used by TA_BINARY_ADD_SCALED */
} ta_epilogue;

/* ref tensor_ash.h:61-65. */
typedef struct ta_matmul_op {
  ta_matmul_call call;
  ta_epilogue epilogue;
} ta_matmul_op;

/* ref tensor_ash.h:67-74. */
enum {
  TA_SOFTMAX_MASK_FULL = 0,
  TA_SOFTMAX_MASK_PREFIX = 1,
  TA_SOFTMAX_MASK_CAUSAL = 2
};

/* ref tensor_ash.h:76-85. */
typedef struct ta_rope_desc {
  uint32_t heads;
  uint32_t head_dim;
  uint32_t rot_dim;
  uint32_t pos_base;
} ta_rope_desc;

/* ref tensor_ash.h:87-94. */
typedef struct ta_copy_desc {
  uint32_t extent[3];
  uint32_t src_offset;
  uint32_t src_strides[3];
  uint32_t dst_offset;
  uint32_t dst_strides[3];
} ta_copy_desc;

/* ref tensor_ash.h:96-104. */
typedef struct ta_dispatch_info {
  const char *kernel;
  uint32_t tile[3];
  uint32_t has_split_k2;
  uint32_t split_k2_splits;
} ta_dispatch_info;

const char *ta_version(void);    /* ref tensor_ash.h:106 */
const char *ta_last_error(void); /* ref tensor_ash.h:107 */

/* ref tensor_ash.h:109-111.  device_preference: NULL/"auto"/"discrete"
 * (HIP device 0), "N" or "index:N", "name:<substr>" or "<substr>"
 * matched against the device name and gfx arch. */
ta_context *ta_context_create(uint32_t enable_validation,
                              const char *device_preference);
void ta_context_destroy(ta_context *ctx); /* ref tensor_ash.h:112 */

/* ref tensor_ash.h:114-116: 1 on HIP devices, 0 for null. */
uint32_t ta_context_supports_f16(const ta_context *ctx);
uint32_t ta_context_supports_bda(const ta_context *ctx);

/* ref tensor_ash.h:118-120.  kernel_selection: NULL/"auto" or an
 * ML_KERNEL name (see ta_kernel_name). */
ta_executor *ta_executor_create(const ta_context *ctx, size_t n_slots,
                                uint32_t max_calls_per_submit,
                                const char *kernel_selection);
/* ref tensor_ash.h:121-129. */
ta_executor *ta_executor_create_v2(const ta_context *ctx, size_t n_slots,
                                   uint32_t max_calls_per_submit,
                                   const char *kernel_selection,
                                   uint32_t tune);
void ta_executor_destroy(ta_executor *exec); /* ref tensor_ash.h:130 */

/* ref tensor_ash.h:132-145. */
ta_tensor *ta_tensor_create(const ta_context *ctx, const uint32_t *shape,
                            size_t rank);
ta_tensor *ta_tensor_create_on_executor(const ta_executor *exec,
                                        const uint32_t *shape, size_t rank);
ta_tensor *ta_tensor_create_f16(const ta_context *ctx, const uint32_t *shape,
                                size_t rank);
ta_tensor *ta_tensor_create_f16_on_executor(const ta_executor *exec,
                                            const uint32_t *shape, size_t rank);
void ta_tensor_destroy(ta_tensor *tensor);          /* ref :146 */
uint64_t ta_tensor_len(const ta_tensor *tensor);        /* ref :147 */
uint64_t ta_tensor_size_bytes(const ta_tensor *tensor); /* ref :148 */
uint32_t ta_tensor_is_f16(const ta_tensor *tensor);     /* ref :149 */

/* ref tensor_ash.h:151-154.  f32 host data; f16 tensors round (RNE) on
 * upload and widen on download. */
int ta_upload(const ta_executor *exec, const ta_tensor *dst, const float *src,
              size_t len);
int ta_download(const ta_executor *exec, const ta_tensor *src, float *dst,
                size_t len);

/* ref tensor_ash.h:156-160. */
int ta_matmul(const ta_executor *exec, const ta_tensor *a, const ta_tensor *b,
              const ta_tensor *c, float alpha, uint32_t accumulate,
              ta_run_stats *stats);
int ta_matmul_batch(const ta_executor *exec, const ta_matmul_call *calls,
                    size_t n_calls, ta_run_stats *stats);

/* ref tensor_ash.h:162-165: independent ops, one submission. */
int ta_run_ops(const ta_executor *exec, const ta_matmul_op *ops, size_t n_ops,
               ta_run_stats *stats);
/* ref tensor_ash.h:166-170: dependent chain, one submission. */
int ta_run_op_graph(const ta_executor *exec, const ta_matmul_op *ops,
                    size_t n_ops, ta_run_stats *stats);

/* ref tensor_ash.h:172-208: model ops (src/executor/elementwise/ops.rs),
 * with the reference's validations and error texts. */
int ta_softmax_rows(const ta_executor *exec, const ta_tensor *input,
                    const ta_tensor *output, float scale, uint32_t mask_kind,
                    uint32_t valid_or_prefix, uint32_t rows_per_group,
                    ta_run_stats *stats);
int ta_rms_norm(const ta_executor *exec, const ta_tensor *input,
                const ta_tensor *weight, const ta_tensor *output, float eps,
                ta_run_stats *stats);
int ta_layer_norm(const ta_executor *exec, const ta_tensor *input,
                  const ta_tensor *weight, const ta_tensor *bias,
                  const ta_tensor *output, float eps, ta_run_stats *stats);
int ta_rope(const ta_executor *exec, const ta_tensor *input,
            const ta_tensor *table, const ta_tensor *output,
            const ta_rope_desc *desc, ta_run_stats *stats);
int ta_copy_strided(const ta_executor *exec, const ta_tensor *src,
                    const ta_tensor *dst, const ta_copy_desc *desc,
                    ta_run_stats *stats);

/* ref tensor_ash.h:210-233: validate, route and record once (a hipGraph),
 * replay with one launch per call.  The executor and every tensor must
 * outlive the handle; destroy waits for in-flight work. */
ta_prepared *ta_prepared_create(const ta_executor *exec,
                                const ta_matmul_op *ops, size_t n_ops,
                                uint32_t as_graph);
int ta_prepared_run(ta_prepared *prepared, ta_run_stats *stats);
int ta_prepared_submit(ta_prepared *prepared);
int ta_prepared_wait(ta_prepared *prepared, ta_run_stats *stats);
void ta_prepared_destroy(ta_prepared *prepared);

/* ref tensor_ash.h:235-240. */
int ta_dispatch_info_for(const ta_executor *exec, uint32_t batch, uint32_t m,
                         uint32_t n, uint32_t k, uint32_t b_f16,
                         ta_dispatch_info *out);
/* ref tensor_ash.h:241-244. */
int ta_tune_shape(const ta_executor *exec, uint32_t batch, uint32_t m,
                  uint32_t n, uint32_t k);

/* ------------------------------------------------------------------ */
/* Additive extensions (no reference C symbol; Rust-API counterparts). */

/* Executor::run_matmuls_split_k2 (src/executor/reduction.rs:21-70):
 * deterministic two-stage split-K.  splits == 0 picks a default;
 * accumulate is not supported. */
int ta_matmul_split_k2(const ta_executor *exec, const ta_tensor *a,
                       const ta_tensor *b, const ta_tensor *c, float alpha,
                       uint32_t splits, ta_run_stats *stats);

/* Executor::run_op_split_k2: ta_matmul_split_k2 for a whole op.  Stage 1
 * writes alpha-scaled partial planes, the reduce sums them in a fixed
 * order and then applies the op's epilogue once (accumulate, bias,
 * activation, binary with D, in the order of ref tensor_ash.h:47-59), so
 * the result is bit-identical from run to run.  No reference symbol: the
 * reference splits plain calls only (src/executor/mod.rs:179-210,
 * shaders/matmul_f32_splitk2_reduce.comp:44-75); ta_run_ops takes this
 * route by itself for deep-K f32 ops whose tiles leave most CUs idle.
 * splits == 0 picks the default; splits == 1 is the data-parallel route. */
int ta_run_op_split_k2(const ta_executor *exec, const ta_matmul_op *op,
                       uint32_t splits, ta_run_stats *stats);

/* No counterpart in the reference.  For callers that cannot allocate
 * device memory (tight serving loops, harnesses that forbid hipMalloc):
 * ta_matmul_split_k2 with the same kernels and bit-identical results at
 * every split count (splits == 1 included: the same data-parallel route),
 * but its partial planes live in a fixed per-device array of
 * TA_NOALLOC_SCRATCH_BYTES that the library holds until the process
 * ends, so the call allocates nothing (ta_allocation_count is unchanged
 * across it).  It runs on the executor's own stream and waits for it, so
 * it is not a call to make inside a caller's stream capture.  Fails
 * (-1, ta_last_error) when the planes would exceed that size: batch * M *
 * N * splits * sub-windows * 4 bytes, where the library adds sub-windows
 * to fill the device (64x256 and 32x128 outputs use 16 MiB and 4 MiB at
 * any split count).  Calls on one device share the array; the library
 * serialises them within a process, and the array keeps the last call's
 * partials. */
#define TA_NOALLOC_SCRATCH_BYTES (32u << 20)
int ta_matmul_split_k2_noalloc(const ta_executor *exec, const ta_tensor *a,
                               const ta_tensor *b, const ta_tensor *c,
                               float alpha, uint32_t splits,
                               ta_run_stats *stats);

/* No counterpart in the reference (a diagnostic): the number of device
 * and pinned-host allocations the library has made in this process
 * (tensors, cells, executor scratch).  Unchanged across a call that
 * allocates nothing. */
uint64_t ta_allocation_count(void);

/* MatmulOp::with_packed_b (src/matmul/api.rs:260-265): B holds the packed
 * decode layout produced by ta_pack_f16w_row_tiles with
 * ta_f16w_row_tile_n(K, N).  Packed ops take M <= 8, batch 1, f16 B. */
typedef struct ta_matmul_op_v2 {
  ta_matmul_op base;
  uint32_t packed_b;
  uint32_t reserved[3]; /* must be zero */
} ta_matmul_op_v2;
int ta_run_ops_v2(const ta_executor *exec, const ta_matmul_op_v2 *ops,
                  size_t n_ops, ta_run_stats *stats);
int ta_run_op_graph_v2(const ta_executor *exec, const ta_matmul_op_v2 *ops,
                       size_t n_ops, ta_run_stats *stats);
ta_prepared *ta_prepared_create_v2(const ta_executor *exec,
                                   const ta_matmul_op_v2 *ops, size_t n_ops,
                                   uint32_t as_graph);

/* Decode fusions of MatmulOp (src/matmul/api.rs:107-299), which the
 * reference exposes in its Rust API only (MatmulOp::with_normed_a,
 * with_store_rope, with_store_scatter, with_store_rope_scatter):
 *  - norm_weight != NULL: C = rms_norm(A, norm_weight, norm_eps) @ B on a
 *    decode GEMV route (M <= 8, batch 1); excludes an epilogue bias and
 *    the add_scaled binary;
 *  - store_kind (M = 1, f16 B, no epilogue, no accumulate): RoPE-rotate
 *    the output row and store it to C, and/or scatter it into store_dst
 *    (f32 or f16) at P * pos_scale + (c / head_dim) * stride_head +
 *    (c % head_dim) * stride_dim, P = pos_base + *pos_addr (pos_addr: a
 *    device address from ta_tensor_device_address, or 0). */
enum {
  TA_STORE_NONE = 0,
  TA_STORE_ROPE = 1,
  TA_STORE_SCATTER = 2,
  TA_STORE_ROPE_SCATTER = 3,
};
typedef struct ta_store_desc { /* MatmulStoreDesc, src/matmul/api.rs:117-133 */
  uint32_t head_dim;
  uint32_t pos_base;
  uint32_t pos_scale;
  uint32_t stride_head;
  uint32_t stride_dim;
  uint32_t reserved; /* must be zero */
  uint64_t pos_addr;
} ta_store_desc;
typedef struct ta_matmul_op_v3 {
  ta_matmul_op_v2 v2;
  const ta_tensor *norm_weight; /* f32 [K], or NULL */
  float norm_eps;
  uint32_t store_kind;          /* TA_STORE_* */
  const ta_tensor *store_table; /* f32 [T_max, head_dim/2, 2] (rope kinds) */
  const ta_tensor *store_dst;   /* scatter kinds */
  ta_store_desc store;
} ta_matmul_op_v3;
int ta_run_ops_v3(const ta_executor *exec, const ta_matmul_op_v3 *ops,
                  size_t n_ops, ta_run_stats *stats);
int ta_run_op_graph_v3(const ta_executor *exec, const ta_matmul_op_v3 *ops,
                       size_t n_ops, ta_run_stats *stats);
ta_prepared *ta_prepared_create_v3(const ta_executor *exec,
                                   const ta_matmul_op_v3 *ops, size_t n_ops,
                                   uint32_t as_graph);
/* Tensor::device_address (src/tensor.rs): the allocation's device address
 * (0 for NULL), e.g. for ta_store_desc.pos_addr. */
uint64_t ta_tensor_device_address(const ta_tensor *tensor);

/* Causal prefill attention, Executor::run_flash_attention
 * (src/executor/elementwise/flash.rs:13-250; FlashAttentionDesc,
 * src/executor/elementwise/mod.rs:160-184), which the reference exposes
 * in its Rust API only.  out = softmax_causal(q Kt * scale) V in one
 * launch: query row i attends to cache positions < min(kv_len, pos_base
 * + i + 1).  kt is [H_kv, dh, T_max], v is [H_kv, T_max, dh] (f32 or
 * f16, alike), dh 64 or 128, H a multiple of H_kv.  q/out are f32, or
 * f16 with f16 caches; head-major [H, T, dh] unless token_major_heads
 * (q, and out unless out_token_major_heads) is nonzero: token-major
 * [T, H*dh]. */
typedef struct ta_flash_desc {
  uint32_t kv_len;
  uint32_t pos_base;
  float scale;                    /* 1/sqrt(dh) for standard attention */
  uint32_t token_major_heads;     /* 0: q is head-major */
  uint32_t out_token_major_heads; /* 0: out follows q */
  uint32_t reserved;              /* must be zero */
} ta_flash_desc;
int ta_flash_attention(const ta_executor *exec, const ta_tensor *q,
                       const ta_tensor *kt, const ta_tensor *v,
                       const ta_tensor *out, const ta_flash_desc *desc,
                       ta_run_stats *stats);

/* Fused RoPE + strided scatter, Executor::run_rope_scatter
 * (src/executor/elementwise/ops.rs:243-316; RopeScatterDesc,
 * src/executor/elementwise/mod.rs:144-159; Rust API only in the
 * reference): ta_rope's rotation of f32 input [T, heads, head_dim], every
 * element (t, h, d) written to dst[dst_offset + t*dst_strides[0] +
 * h*dst_strides[1] + d*dst_strides[2]] (dst f32, or f16 with RNE; not the
 * input).  pos_scale applies when a graph op carries a position cell. */
typedef struct ta_rope_scatter_desc {
  uint32_t dst_offset;
  uint32_t dst_strides[3];
  uint32_t pos_scale;
  uint32_t reserved; /* must be zero */
} ta_rope_scatter_desc;
int ta_rope_scatter(const ta_executor *exec, const ta_tensor *input, const ta_tensor *table,
                    const ta_tensor *dst, const ta_rope_desc *desc,
                    const ta_rope_scatter_desc *scatter, ta_run_stats *stats);

/* Binary combine, Executor::run_binary (ops.rs:318-380; BinaryOp,
 * elementwise/mod.rs:242-252; Rust API only in the reference): over
 * equal-length a, b, out (all f32 or all f16; out may alias a or b),
 * TA_BINARY_OP_ADD_SCALED: out = a + beta * b; TA_BINARY_OP_SILU_MUL: out =
 * silu(a) * b (beta ignored). */
enum { TA_BINARY_OP_ADD_SCALED = 0, TA_BINARY_OP_SILU_MUL = 1 };
int ta_binary(const ta_executor *exec, const ta_tensor *a, const ta_tensor *b,
              const ta_tensor *out, uint32_t op, float beta, ta_run_stats *stats);

/* Prefill QKV pack, Executor::run_prefill_qkv_pack
 * (src/executor/elementwise/flash.rs:255-402; PrefillQkvPackDesc,
 * elementwise/mod.rs:186-199; Rust API only in the reference): from f16 qkv
 * [T, H*dh + 2*H_kv*dh], RoPE Q into head-major f16 q [H, T, dh], RoPE K
 * into the f16 Kt cache [H_kv, dh, T_max] and copy V into the f16 V cache
 * [H_kv, T_max, dh], both at positions pos_base .. pos_base + T - 1; table
 * f32 [T_max, rot_dim/2, 2]; dh a multiple of 4. */
typedef struct ta_prefill_qkv_pack_desc {
  uint32_t heads, kv_heads, head_dim, rot_dim, pos_base;
  uint32_t reserved; /* must be zero */
} ta_prefill_qkv_pack_desc;
int ta_prefill_qkv_pack(const ta_executor *exec, const ta_tensor *qkv, const ta_tensor *table,
                        const ta_tensor *q, const ta_tensor *kt, const ta_tensor *v,
                        const ta_prefill_qkv_pack_desc *desc, ta_run_stats *stats);

/* Executor::run_gemv_chain (src/executor/elementwise/gemv_chain.rs:14-194;
 * Rust API only in the reference): up to TA_GEMV_CHAIN_MAX_JOBS M = 1 row
 * GEMVs on row-major f16 B (f32 A and C; no bias, store, accumulate or
 * packed B; activation none or SiLU; normed-A not with AddScaled), run in
 * list order. */
#define TA_GEMV_CHAIN_MAX_JOBS 8
int ta_run_gemv_chain(const ta_executor *exec, const ta_matmul_op_v3 *jobs, size_t n_jobs,
                      ta_run_stats *stats);

/* Host-visible u32 cells (src/executor/cells.rs:10-205; Rust API only in
 * the reference): pinned, mapped host memory that kernels read and write
 * through ta_u32_cell_device_address and the host through
 * ta_u32_cell_write / ta_u32_cell_read between submissions.  cap 1 plays
 * PosBuffer (create_pos_buffer) and HostU32Buffer
 * (create_host_u32_buffer); cap n plays TokenIdBuffer
 * (create_token_id_buffer).  Cells start zeroed.  ta_u32_cell_write fails
 * when n exceeds cap; ta_u32_cell_read returns element 0. */
typedef struct ta_u32_cell ta_u32_cell;
ta_u32_cell *ta_u32_cell_create(ta_context *ctx, uint32_t cap);
void ta_u32_cell_destroy(ta_u32_cell *cell);
int ta_u32_cell_write(ta_u32_cell *cell, const uint32_t *values, size_t n);
int ta_u32_cell_read(const ta_u32_cell *cell, uint32_t *value);
uint64_t ta_u32_cell_device_address(const ta_u32_cell *cell);
uint32_t ta_u32_cell_cap(const ta_u32_cell *cell);

/* The GPU token loop, Executor::run_argmax / run_embed_gather /
 * run_embed_gather_rows (src/executor/elementwise/ops.rs:456-595; Rust
 * API only in the reference).  ta_argmax writes to element 0 of `result`
 * the index of the largest value of `input` (f32, any shape, read flat),
 * the largest index among equal maxima (the reference's greedy sampler).
 * ta_embed_gather copies row min(tokens[t], vocab - 1) of `table`
 * ([vocab, embd], f32 or f16) to row t of `out` ([embd] or [t, embd], f32
 * or f16), reading the ids when the op runs, so it can follow ta_argmax in
 * a graph with no host round trip. */
int ta_argmax(const ta_executor *exec, const ta_tensor *input, ta_u32_cell *result,
              ta_run_stats *stats);
int ta_embed_gather(const ta_executor *exec, const ta_u32_cell *tokens,
                    const ta_tensor *table, const ta_tensor *out, ta_run_stats *stats);

/* Fused split-K decode attention, Executor::run_attn_decode
 * (src/executor/elementwise/attn.rs:14-185; AttnDecodeDesc,
 * src/executor/elementwise/mod.rs:200-241; Rust API only in the
 * reference): out = softmax(q Kt * scale) V for one query row per head
 * over the kv_len valid cache positions (never reading past them).  q and
 * out are f32 [kv_heads, group, dh] (group <= 8), kt [kv_heads, dh,
 * T_max], v [kv_heads, T_max, dh] (f32 or f16, alike), dh 64 or 128.
 * scratch (f32) holds at least kv_heads * TA_ATTN_DECODE_MAX_CHUNKS *
 * group * (dh + 2) values.  pos_addr (device address of a u32 cell, 0 =
 * none) adds the cell's value to kv_len when the op runs. */
#define TA_ATTN_DECODE_MAX_CHUNKS 32
typedef struct ta_attn_decode_desc {
  uint32_t kv_len;
  float scale; /* 1/sqrt(dh) for standard attention */
  uint64_t pos_addr;
} ta_attn_decode_desc;
int ta_attn_decode(const ta_executor *exec, const ta_tensor *q, const ta_tensor *kt,
                   const ta_tensor *v, const ta_tensor *scratch, const ta_tensor *out,
                   const ta_attn_decode_desc *desc, ta_run_stats *stats);

/* Mixed-op graphs, Executor::run_exec_ops / prepare_exec_ops with ExecOp
 * (src/executor/graph_ops.rs:23-336), Rust-API-only in the reference: a
 * dependent chain of matmuls and model ops run (or recorded once as a
 * hipGraph) in list order, every op seeing all earlier writes; every op
 * is validated before anything is launched.  Operand roles by kind:
 *   MATMUL          matmul (in/out unused)
 *   RMS_NORM        in[0] input, in[1] weight, out; scalar = eps
 *   LAYER_NORM      in[0] input, in[1] weight, in[2] bias, out; scalar = eps
 *   SOFTMAX_ROWS    in[0] input, out; scalar = scale; mask_kind,
 *                   valid_or_prefix, rows_per_group as ta_softmax_rows
 *   ROPE            in[0] input, in[1] table, out; rope
 *   COPY_STRIDED    in[0] src, out dst; copy
 *   FLASH_ATTENTION in[0] q, in[1] kt, in[2] v, out; flash
 *   ARGMAX          in[0] input; cell result
 *   EMBED_GATHER    cell token ids, in[0] table, out
 *   ATTN_DECODE     in[0] q, in[1] kt, in[2] v, aux scratch, out; attn
 *   ROPE_SCATTER    in[0] input, in[1] table, out dst; rope, scatter
 *                   (pos_addr as for ROPE, advancing dst by
 *                   scatter.pos_scale per position)
 *   BINARY          in[0] a, in[1] b, out; binary_op, scalar = beta
 *   PREFILL_QKV_PACK in[0] qkv, in[1] table, out q, aux kt, aux2 v; qkv
 *   GEMV_CHAIN      matmul -> n_jobs jobs (ta_run_gemv_chain's rules)
 * pos_addr (ROPE, COPY_STRIDED): device address of a u32 position cell
 * read when the op runs (added to rope.pos_base; times pos_scale added to
 * copy.dst_offset), so a prepared graph replays at a new position after
 * the cell is rewritten; 0 = none. */
enum {
  TA_EXEC_MATMUL = 0,
  TA_EXEC_RMS_NORM = 1,
  TA_EXEC_LAYER_NORM = 2,
  TA_EXEC_SOFTMAX_ROWS = 3,
  TA_EXEC_ROPE = 4,
  TA_EXEC_COPY_STRIDED = 5,
  TA_EXEC_FLASH_ATTENTION = 6,
  TA_EXEC_ARGMAX = 7,
  TA_EXEC_EMBED_GATHER = 8,
  TA_EXEC_ATTN_DECODE = 9,
  TA_EXEC_ROPE_SCATTER = 10,
  TA_EXEC_BINARY = 11,
  TA_EXEC_PREFILL_QKV_PACK = 12,
  TA_EXEC_GEMV_CHAIN = 13,
};
typedef struct ta_exec_op {
  uint32_t kind; /* TA_EXEC_* */
  uint32_t mask_kind;
  uint32_t valid_or_prefix;
  uint32_t rows_per_group;
  float scalar;
  uint32_t pos_scale;
  uint64_t pos_addr;
  const ta_tensor *in[3];
  const ta_tensor *out;
  const ta_matmul_op_v3 *matmul;
  ta_rope_desc rope;
  ta_copy_desc copy;
  ta_flash_desc flash;
  const ta_u32_cell *cell;
  const ta_tensor *aux;
  ta_attn_decode_desc attn;
  const ta_tensor *aux2;
  ta_rope_scatter_desc scatter;
  uint32_t binary_op; /* TA_BINARY_OP_* */
  ta_prefill_qkv_pack_desc qkv;
  uint32_t n_jobs; /* GEMV_CHAIN */
} ta_exec_op;
int ta_run_exec_ops(const ta_executor *exec, const ta_exec_op *ops,
                    size_t n_ops, ta_run_stats *stats);
ta_prepared *ta_prepared_create_exec(const ta_executor *exec,
                                     const ta_exec_op *ops, size_t n_ops);

/* pack_f16w_row_tiles (src/matmul/api.rs:324-344): row-major [K, N] ->
 * [N/tile_n][K][tile_n]; dst holds K*N floats. */
int ta_pack_f16w_row_tiles(const float *src, size_t k, size_t n,
                           size_t tile_n, float *dst);
/* f16w_row_tile_n (src/pipeline/routing.rs:17-23): the packing tile the
 * decode GEMV expects for this shape (64 when N % 64 == 0, else 32). */
uint32_t ta_f16w_row_tile_n(uint32_t k, uint32_t n);

/* Executor::upload_f16 (src/executor/transfer.rs:41-55): raw binary16
 * bits into an f16 tensor. */
int ta_upload_f16(const ta_executor *exec, const ta_tensor *dst,
                  const uint16_t *src, size_t len);

/* KERNEL_SPECS introspection (src/pipeline/catalog.rs:129-197). */
size_t ta_kernel_count(void);
/* Name of registry entry i (NULL past the end); valid for the process. */
const char *ta_kernel_name(size_t index);
/* Tile of entry i into tile[3]; -1 past the end. */
int ta_kernel_tile(size_t index, uint32_t *tile);

/* Device facts for reporting: compute-unit count, or 0 for null. */
uint32_t ta_context_cu_count(const ta_context *ctx);

#ifdef __cplusplus
}
#endif

#endif
