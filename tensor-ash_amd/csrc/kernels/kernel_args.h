// Kernel argument blocks shared by the host runtime and the gfx950 code
// objects.  Every kernel takes exactly one of these structs by value; the
// host passes it through hipModuleLaunchKernel's kernelParams.  Plain C
// layout: no pointers to host memory, no torch or HIP types.
//
// The fields play the role of the reference's 144-byte push-constant block
// (src/pipeline/abi.rs:15-53), laid out for HIP kernargs: 64-bit element
// strides instead of u32 so batched planes past 4 GiB need no special path.
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// Epilogue flag bits (GemmArgs.flags / GemvArgs.flags).
enum {
  TA_FLAG_ACCUMULATE = 1u << 0, // v += C_old (after alpha)
  TA_FLAG_BIAS = 1u << 1,       // v += bias[batch * bias_batch_stride + col]
  TA_GEMV_PACKED = 1u << 2,     // GEMV weights in the [N/TW][K][TW] layout
};

// Bytes of the fixed device scratch that the allocation-free split-K
// entry point keeps its partial planes in (one array per device, held
// until the process ends).  Config 4's largest plane set is 16 MiB.
// The public header states the same figure as TA_NOALLOC_SCRATCH_BYTES;
// capi.cpp, which sees both, asserts that they agree.
#define TA_FIXED_SCRATCH_BYTES (32u << 20)

// Most chunks a split-K decode-attention launch uses per kv head: stage 2
// (ta_attn_decode_combine) keeps one register slot per chunk and one LDS
// weight per lane, so the cap must stay <= 64 (the wave width).
#define TA_ATTN_DECODE_MAX_CHUNKS 32

// Activation codes (shaders/matmul_epilogue_common.glsl:24-26 numbering).
enum { TA_ACT_NONE = 0, TA_ACT_RELU = 1, TA_ACT_SILU = 2, TA_ACT_GELU = 3 };
// Binary codes: 1 = += beta * D, 2 = *= D.
enum { TA_BIN_NONE = 0, TA_BIN_ADD_SCALED = 1, TA_BIN_MUL = 2 };

// Dense GEMM: C[b] = epilogue(alpha * A[b] @ B[b] (+ C[b])).
// A is [M, K] row-major, B is [K, N] row-major (f32 or f16 storage),
// C and D are [M, N] row-major f32.  A stride of 0 broadcasts one plane.
// Split-K stage 1 (num_splits > 1): grid.z = batch * num_splits, split s
// of batch b owns its K window and stores alpha * partial to plane
// (b * num_splits + s) of `c` (the scratch), with no epilogue.
typedef struct GemmArgs {
  const void *a;
  const void *b;
  float *c;
  const float *d;
  const float *bias;
  uint64_t stride_a; // elements between batch planes (0 = broadcast)
  uint64_t stride_b;
  uint64_t stride_c;
  uint32_t m, n, k;
  uint32_t flags;
  uint32_t act;
  uint32_t binary;
  uint32_t bias_batch_stride; // 0 for [N] bias, N for [B, N]
  uint32_t num_splits;        // partial planes per batch (S * sub_splits); 1 = plain GEMM
  float alpha;
  float beta;
  uint32_t tiles_n; // ceil(N / BN): for the blockIdx -> tile remap
  uint32_t tiles_m; // ceil(M / BM)
  // Split-K: each of the S = num_splits / sub_splits splits owns the
  // reference window of K, cut again into sub_splits windows by the same
  // rule; plane (batch * num_splits + s * sub_splits + t) holds window t of
  // split s.
  uint32_t sub_splits;
  // In-kernel split-K (ta_gemm_h16sk_*): k_splits workgroups share each
  // output tile, each over its K window (blockIdx.y = split); they store
  // their f32 partial tiles to `partial` ((batch tile * k_splits + split)
  // * BM * BN floats), count themselves in counters[batch tile *
  // TA_GEMV_COUNTER_STRIDE], and the last to arrive sums the partials in
  // split order, applies the epilogue and resets the counter to zero.
  uint32_t k_splits;
  float *partial;
  uint32_t *counters;
  // Dual SwiGLU launch (ta_gemm_h16dual_*): second weight matrix (same
  // shape and strides as b) and the output U = alpha * A @ b2 goes to c2;
  // the launch's own epilogue has binary Mul with d = c2.
  const void *b2;
  float *c2;
  // Optional f16 (RNE) copy of the final C values, same layout as c (f32-C
  // launches without split planes); null = none.  Lets a following f16w
  // GEMM that reads this C as A skip its conversion pre-pass.
  uint16_t *c16;
} GemmArgs;

// Fixed-order reduction of split-K partial planes:
// C[b][e] = sum_{s=0}^{S-1} scratch[(b * S + s) * mn + e].
// The sum then takes the op's fused epilogue without alpha, which stage 1
// already applied to every partial: v = sum (+C_old) -> +bias -> act ->
// (+beta*D | *D); flags / act / binary / beta take GemmArgs' meaning.
typedef struct SplitReduceArgs {
  const float *scratch;
  float *c;
  uint64_t total; // batch * mn
  uint64_t mn;
  uint32_t num_splits;
  uint32_t groups; // plane groups per element: power of two <= min(num_splits, 256)
  const float *bias;
  const float *d;
  uint32_t n; // columns of C (epilogue column = (e % mn) % n)
  uint32_t flags;
  uint32_t act;
  uint32_t binary;
  uint32_t bias_batch_stride;
  float beta;
} SplitReduceArgs;

// Element-wise f32 -> f16 (RNE) conversion: dst[i] = src[i], i < n.
typedef struct CvtArgs {
  const float *src;
  uint16_t *dst;
  uint64_t n;
} CvtArgs;

// Two conversions in one launch: blocks [0, blocks0) convert job[0], the
// rest job[1] (the inputs a submission's f16w GEMMs convert, up front).
typedef struct CvtPairArgs {
  CvtArgs job[2];
  uint64_t blocks0;
} CvtPairArgs;

// Decode GEMV over packed f16 weights W[N/TW][K][TW] (or row-major):
// Y[m, :] = epilogue(alpha * X[m, :] @ W) for m < rows (rows <= 8).
// With `w2` set (dual mode) the same launch also computes
// U = alpha * X @ W2, stores U to `y2` and Y = act(alpha * X @ W + bias) * U
// to `y` (SwiGLU gating); then `binary` must be TA_BIN_NONE.
// K is cut into `kchunks` windows of `kchunk` rows; every (tile, window)
// workgroup stores its partial to `partial`, and the last workgroup of a
// tile to arrive (counted in `counters[tile * stride]`) sums the windows in
// window order and applies the epilogue.  That workgroup resets the
// counter, so the buffer stays zero between launches.

// One counter or flag per 128-byte line (atomics on a shared line
// serialise across tiles).
#define TA_GEMV_COUNTER_STRIDE 32u

typedef struct GemvArgs {
  const float *x; // [rows, K] f32
  const uint16_t *w;
  const uint16_t *w2;
  float *y;  // [rows, N]
  float *y2; // dual mode only
  const float *d;
  const float *bias;
  float *partial;     // [kchunks][tiles][ways][MR][TW]
  uint32_t *counters; // [tiles * TA_GEMV_COUNTER_STRIDE]
  uint32_t rows, n, k;
  uint32_t kchunk;
  uint32_t kchunks;
  uint32_t flags;
  uint32_t act;
  uint32_t binary;
  float alpha;
  float beta;
} GemvArgs;

// Decode fusions of a standalone GEMV launch (its second kernel argument;
// src/matmul/api.rs:107-299 semantics):
//  * norm_w != null: RMSNorm of every X row folded in before the product,
//    X'[m, k] = (X[m, k] * s_m) * norm_w[k], s_m = 1 / sqrt(mean_k X[m, k]^2
//    + norm_eps);
//  * store_mode (M = 1): 1 = RoPE-rotate the output pairs and store to Y,
//    2 = scatter Y into store_dst, 3 = rotate then scatter (Y untouched in
//    modes 2 and 3).  Position P = pos_base + (pos_addr ? *pos_addr : 0).
typedef struct GemvFusion {
  const float *norm_w;
  float norm_eps;
  uint32_t store_mode;
  uint32_t store_dst_f16;
  uint32_t head_dim;
  uint32_t pos_base;
  uint32_t pos_scale;
  uint32_t stride_head;
  uint32_t stride_dim;
  const uint32_t *pos_addr;
  const float *rope_table; // [T_max, head_dim / 2, 2] (cos, sin)
  void *store_dst;         // f32 or f16 elements
  // Element counts of rope_table / store_dst: a device position that
  // reaches past them skips the element instead of reading or writing
  // out of bounds.
  uint64_t table_len, dst_len;
} GemvFusion;

// Persistent GEMV chain (ta_gemv_chain_f16_m1; the reference's GemvChain,
// src/executor/elementwise/gemv_chain.rs): up to TA_GEMV_CHAIN_MAX_JOBS
// M = 1 GEMVs with row-major f16 weights (64-column tiles) in one launch.  Jobs run in
// groups: consecutive jobs without a data hazard share one grid-stride
// space of units (tile, K window), and a group that a later job depends on
// (bit j of sync_after: the group ending at job j) is followed by a grid
// barrier.  A unit is exactly a standalone GEMV workgroup (same K windows,
// same fixed-order window reduction through job[j].partial / .counters,
// same epilogue), so the results equal the jobs' standalone launches.
#define TA_GEMV_CHAIN_MAX_JOBS 8
typedef struct GemvChainArgs {
  GemvArgs job[TA_GEMV_CHAIN_MAX_JOBS];
  GemvFusion fu[TA_GEMV_CHAIN_MAX_JOBS];
  uint32_t units[TA_GEMV_CHAIN_MAX_JOBS]; // ceil(n / 64) tiles * kchunks
  uint32_t n_jobs;
  uint32_t sync_after;
  uint32_t spin_limit; // barrier polls before a wait gives up
  uint32_t pad;
  uint32_t *barrier;   // [2 * TA_GEMV_COUNTER_STRIDE]: arrivals, generation (zeroed once)
  uint32_t *status;    // host-mapped; set to 1 if a wait gave up (results invalid)
} GemvChainArgs;

// ---- model ops (ta_softmax_rows, ta_rms_norm, ta_layer_norm, ta_rope,
// ta_copy_strided; src/executor/elementwise/ops.rs semantics) ----

// Row softmax: valid = causal ? min(cols, valid_base + row % rows_per_group
// + 1) : min(cols, valid_base); columns >= valid store 0.
typedef struct SoftmaxArgs {
  const float *in;
  float *out;
  uint32_t rows, cols;
  uint32_t valid_base, rows_per_group, causal;
  float scale;
} SoftmaxArgs;

// Row norm: RMSNorm (bias null) or LayerNorm; io_f16: f16 input/output.
typedef struct NormArgs {
  const void *in;
  void *out;
  const float *weight;
  const float *bias;
  uint32_t rows, cols;
  float eps;
  uint32_t io_f16;
} NormArgs;

// RoPE over [tokens, heads, head_dim]: pairs (2i, 2i+1) of the first
// rot_dim lanes rotate by table[(pos_base + *pos_addr + token) * rot_dim/2
// + i] (cos, sin); the other lanes pass through.
typedef struct RopeArgs {
  const void *in;
  void *out;
  const float *table;
  const uint32_t *pos_addr; // null: none
  uint32_t tokens, heads, head_dim, rot_dim, pos_base;
  uint32_t io_f16;
  uint64_t table_len; // elements; pairs whose angle lies past it are skipped
} RopeArgs;

// Fused RoPE + strided scatter: the rotation of RopeArgs (f32 input),
// every element (token, head, dim) of the rotated [tokens, heads, head_dim]
// vectors written to dst[dst_offset + *pos_addr * pos_scale + token * ds0 +
// head * ds1 + dim * ds2] (f32, or f16 with RNE); destinations past
// dst_len are skipped.
typedef struct RopeScatterArgs {
  RopeArgs rope; // in, table, pos_addr, geometry (out and io_f16 unused)
  void *dst;
  uint32_t dst_offset;
  uint32_t dst_strides[3];
  uint32_t pos_scale;
  uint32_t dst_f16;
  uint64_t dst_len;
} RopeScatterArgs;

// Elementwise combine over n elements: mode 0 out = a + beta * b, mode 1
// out = silu(a) * b; a, b, out all f32 or all f16 (f32 math, RNE store).
typedef struct BinaryArgs {
  const void *a;
  const void *b;
  void *out;
  uint64_t n;
  uint32_t mode;
  float beta;
  uint32_t io_f16;
  uint32_t pad;
} BinaryArgs;

// Prefill QKV pack (f16): from qkv [tokens, qkv_stride] = [Q (heads*dh) |
// K (kv_heads*dh) | V (kv_heads*dh)] per token, RoPE Q into head-major
// q [heads, tokens, dh], RoPE K into kt [kv_heads, dh, t_max] at column
// pos_base + token, copy V into v [kv_heads, t_max, dh] at row pos_base +
// token.  Lanes past rot_dim pass through.
typedef struct QkvPackArgs {
  const uint16_t *qkv; // f16 bits throughout
  uint16_t *q;
  uint16_t *kt;
  uint16_t *v;
  const float *table;
  uint32_t tokens, heads, kv_heads, head_dim, rot_dim, pos_base;
  uint32_t qkv_stride, t_max, k_offset, v_offset;
} QkvPackArgs;

// Strided 3-D copy: for (x, y, z) < extent, dst[dst_offset + *pos_addr *
// pos_scale + x*ds0 + y*ds1 + z*ds2] = src[src_offset + x*ss0 + y*ss1 +
// z*ss2]; f16 sides widen exactly / narrow with RNE.
typedef struct CopyArgs {
  const void *src;
  void *dst;
  const uint32_t *pos_addr; // null: none
  uint32_t extent[3];
  uint32_t src_offset;
  uint32_t src_strides[3];
  uint32_t dst_offset;
  uint32_t dst_strides[3];
  uint32_t pos_scale;
  uint32_t src_f16, dst_f16;
  uint64_t dst_len; // elements; destinations past it are skipped
} CopyArgs;

// Causal prefill attention (one launch): query row i of head h attends to
// cache positions < min(kv_len, pos_base + i + 1) of kv head h /
// group_size.  q/out element (h, i, d) sits at h * head_stride + i *
// row_stride + d; kt is [H_kv, dh, t_max], v is [H_kv, t_max, dh].  The
// grid is q_tiles * heads workgroups of 64 query rows.
typedef struct FlashArgs {
  const void *q;
  const void *kt;
  const void *v;
  void *out;
  uint32_t t_q, t_max, kv_len, pos_base, group_size;
  float scale;
  uint32_t q_head_stride, q_row_stride, o_head_stride, o_row_stride;
  uint32_t heads, q_tiles;
} FlashArgs;

// Greedy-sampling argmax over n f32 values (one workgroup): the index of
// the largest value, the largest index among equal maxima, to *result.
typedef struct ArgmaxArgs {
  const float *in;
  uint32_t *result;
  uint32_t n;
  uint32_t pad;
} ArgmaxArgs;

// Embedding-row gather: out row t = table row min(tokens[t], vocab - 1),
// t < n_tokens; table [vocab, embd] f32 or f16, out [n_tokens, embd] f32 or
// f16.  Grid: (ceil(embd / 1024), n_tokens) workgroups of 256 threads.
typedef struct EmbedArgs {
  const uint32_t *tokens;
  const void *table;
  void *out;
  uint32_t embd, vocab, n_tokens;
  uint32_t table_f16, out_f16;
  uint32_t pad;
} EmbedArgs;

// Split-K decode attention, stage 1: workgroup (chunk, kv_head) attends
// the `group` query rows of kv_head to positions [chunk * cs, min((chunk +
// 1) * cs, L)), cs = ceil(L / num_chunks), L = kv_len (+ *pos when pos is
// set), and stores per row {acc[dh], m, l} (m in log2 units) to
// scratch[kv_head][chunk][row].  q/out [kv_heads, group, dh]; kt [kv_heads,
// dh, t_max]; v [kv_heads, t_max, dh].
typedef struct AttnDecodeArgs {
  const float *q;
  const void *kt;
  const void *v;
  float *scratch;
  const uint32_t *pos;
  uint32_t kv_len, num_chunks, group, t_max;
  float scale;
  uint32_t pad;
} AttnDecodeArgs;

// Stage 2: one workgroup per (kv_head, row) merges the num_chunks
// partials of the row exactly into out[kv_head][row][0..dh).
typedef struct AttnCombineArgs {
  const float *scratch;
  float *out;
  uint32_t num_chunks, group, dh;
  uint32_t pad;
} AttnCombineArgs;

// Persistent decode SwiGLU MLP chain in one launch: `layers` MLPs, layer
// l+1 reading layer l's output y as its x.  In a layer, `a` is the dual
// gate/up GEMV (producer of h = act(x Wg) * (x Wu)) and `b` the down-proj
// GEMV reading h.  Workgroup r serves layer r / (units_a + units_b); within
// a layer the first units_a run `a` units (tile-major: unit u is tile
// u % tiles_a, K window u / tiles_a), the rest `b` units likewise.  Every
// layer has the same shape.
// Units hand data over as 64-bit words {f32 value, tag} that the reader
// polls until the tag matches; layer l's tag is *gen + l + 1, and the last
// tile of the last layer (counted in *done) advances *gen by `layers`, so
// no hand-off word ever needs clearing.  The a/b partial and counters
// fields are unused: the tagged buffers replace them.
#define TA_MLP_MAX_LAYERS 16
// K windows of the decode MLP's two phases: gate/up units take
// TA_MLP_ROWS_A rows of x, down units TA_MLP_ROWS_B rows of h (multiples of
// 256; a unit issues rows / 16 weight loads per lane and matrix).
#ifndef TA_MLP_ROWS_A
#define TA_MLP_ROWS_A 256
#endif
#ifndef TA_MLP_ROWS_B
#define TA_MLP_ROWS_B 256
#endif

typedef struct MlpLayer {
  GemvArgs a;
  GemvArgs b;
} MlpLayer;

typedef struct MlpArgs {
  uint64_t *tag_a;  // [kch_a][tiles_a][2][MR][64] gate/up window partials
  uint64_t *tag_h;  // [K_b][MR] h, as the down units read it
  uint64_t *tag_b;  // [kch_b][tiles_b][MR][64] down window partials
  uint64_t *tag_y;  // [N_b][MR] y, as the next layer's gate/up units read it
  uint32_t *gen;    // launch generation (zero-initialised)
  uint32_t *done;   // last-layer `b` tiles finished (zero between launches)
  uint32_t *status; // host-mapped; set to 1 if a wait gave up
  uint32_t units_a, units_b;
  uint32_t tiles_a, tiles_b;
  uint32_t spin_limit; // polls before a wait gives up
  uint32_t layers;
  // Normed A of the first layer's gate/up (RMSNorm of x folded into their
  // X staging, as in the standalone GEMV); null when x is used as is.
  const float *norm_w;
  float norm_eps;
  uint32_t pad_norm;
  MlpLayer layer[TA_MLP_MAX_LAYERS];
} MlpArgs;

#ifdef __cplusplus
}
#endif

#ifdef __cplusplus
// Work split of the causal prefill attention kernels, shared with the host
// launch (threads = 64 * QB * KP, query tiles of 32 * QB rows).
//   KP: key parts per query block (head dim 64: 4, head dim 128: 2)
//   QB: 32-row query blocks per workgroup
constexpr int ta_flash_parts(int dh) { return dh == 64 ? 4 : 2; }
constexpr int ta_flash_qblocks(int /*dh*/) { return 2; }
constexpr int ta_flash_threads(int dh) { return 64 * ta_flash_qblocks(dh) * ta_flash_parts(dh); }
constexpr int ta_flash_rows(int dh) { return 32 * ta_flash_qblocks(dh); }

// Pipeline stages of the FP32-MFMA (_mi16) kernels: 8 for the 32-row
// tiles (two waves per CU) and the 64 x 64 split-K tile (8 KiB stages), 4
// for the others.  Every K window of a launch must hold a multiple of
// 16 * stages rows.
#ifndef TA_MI16_SKINNY_STAGES
#define TA_MI16_SKINNY_STAGES 8
#endif
constexpr int ta_mi16_stages(int bm, int bn) {
  return bm == 32 || (bm == 64 && bn == 64) ? TA_MI16_SKINNY_STAGES : 4;
}

// Threads of the pipelined f16-MFMA kernels (ta_gemm_{h16,a16}_<tile>_lds,
// ta_gemm_h16sk_<tile>, ta_gemm_h16dual_<tile>_lds): 16 waves (four per
// SIMD, one 32 x 32 block each) for 128 x 128 tiles, 8 waves (two per SIMD)
// for the other tiles of 128 x 64 and larger, 4 waves for 64 x 64.
constexpr int ta_h16_lds_threads(int bm, int bn) {
  return bm == 128 && bn == 128 ? 1024 : bm * bn >= 128 * 64 ? 512 : 256;
}
#endif
