/*
 * A plain C99 caller of include/tensor_ash.h, linked against
 * libtensor_ash.so.  It plays the role of the reference's C example
 * (examples/c_smoke.c:55-104) for this build's tests.
 *
 *   c_caller layout   prints "<struct> <field> <offset> <size>" for every
 *                     field of every struct in the header, then
 *                     "<struct> sizeof <n>" (no GPU needed)
 *   c_caller run      2x3 @ 3x2 = [58, 64, 139, 154], then bias -58.5 +
 *                     SiLU through ta_run_ops, then a prepared replay
 *
 * The _Static_asserts pin the reference structs (ref include/tensor_ash.h:
 * 16-104) to their LP64 layouts, derived from the field lists: any change
 * to the header that moves a field breaks the build of this file.
 */
#include <math.h>
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/tensor_ash.h"

/* ta_run_stats {u32; u64; size_t; u64; double}: 4 + 4 pad, then 8-byte fields. */
_Static_assert(sizeof(ta_run_stats) == 40, "ta_run_stats size");
_Static_assert(offsetof(ta_run_stats, gpu_time_ns) == 8, "gpu_time_ns");
_Static_assert(offsetof(ta_run_stats, n_calls) == 16, "n_calls");
_Static_assert(offsetof(ta_run_stats, total_flops) == 24, "total_flops");
_Static_assert(offsetof(ta_run_stats, tflops) == 32, "tflops");
/* ta_matmul_call {3 pointers; float; u32}. */
_Static_assert(sizeof(ta_matmul_call) == 32, "ta_matmul_call size");
_Static_assert(offsetof(ta_matmul_call, c) == 16, "c");
_Static_assert(offsetof(ta_matmul_call, alpha) == 24, "alpha");
_Static_assert(offsetof(ta_matmul_call, accumulate) == 28, "accumulate");
/* ta_epilogue {pointer; u32; u32; pointer; float + 4 tail pad}. */
_Static_assert(sizeof(ta_epilogue) == 32, "ta_epilogue size");
_Static_assert(offsetof(ta_epilogue, activation) == 8, "activation");
_Static_assert(offsetof(ta_epilogue, binary_kind) == 12, "binary_kind");
_Static_assert(offsetof(ta_epilogue, d) == 16, "d");
_Static_assert(offsetof(ta_epilogue, beta) == 24, "beta");
/* ta_matmul_op {call; epilogue}. */
_Static_assert(sizeof(ta_matmul_op) == 64, "ta_matmul_op size");
_Static_assert(offsetof(ta_matmul_op, epilogue) == 32, "epilogue");
/* ta_rope_desc {4 x u32}. */
_Static_assert(sizeof(ta_rope_desc) == 16, "ta_rope_desc size");
_Static_assert(offsetof(ta_rope_desc, pos_base) == 12, "pos_base");
/* ta_copy_desc {u32[3]; u32; u32[3]; u32; u32[3]}. */
_Static_assert(sizeof(ta_copy_desc) == 44, "ta_copy_desc size");
_Static_assert(offsetof(ta_copy_desc, src_offset) == 12, "src_offset");
_Static_assert(offsetof(ta_copy_desc, src_strides) == 16, "src_strides");
_Static_assert(offsetof(ta_copy_desc, dst_offset) == 28, "dst_offset");
_Static_assert(offsetof(ta_copy_desc, dst_strides) == 32, "dst_strides");
/* ta_dispatch_info {pointer; u32[3]; u32; u32 + 4 tail pad}. */
_Static_assert(sizeof(ta_dispatch_info) == 32, "ta_dispatch_info size");
_Static_assert(offsetof(ta_dispatch_info, tile) == 8, "tile");
_Static_assert(offsetof(ta_dispatch_info, has_split_k2) == 20, "has_split_k2");
_Static_assert(offsetof(ta_dispatch_info, split_k2_splits) == 24, "split_k2_splits");

#define F(S, f) printf("%s %s %zu %zu\n", #S, #f, offsetof(S, f), sizeof(((S *)0)->f))
#define Z(S) printf("%s sizeof %zu\n", #S, sizeof(S))

static void layout(void) {
  F(ta_run_stats, has_gpu_time); F(ta_run_stats, gpu_time_ns); F(ta_run_stats, n_calls);
  F(ta_run_stats, total_flops); F(ta_run_stats, tflops); Z(ta_run_stats);
  F(ta_matmul_call, a); F(ta_matmul_call, b); F(ta_matmul_call, c); F(ta_matmul_call, alpha);
  F(ta_matmul_call, accumulate); Z(ta_matmul_call);
  F(ta_epilogue, bias); F(ta_epilogue, activation); F(ta_epilogue, binary_kind); F(ta_epilogue, d);
  F(ta_epilogue, beta); Z(ta_epilogue);
  F(ta_matmul_op, call); F(ta_matmul_op, epilogue); Z(ta_matmul_op);
  F(ta_rope_desc, heads); F(ta_rope_desc, head_dim); F(ta_rope_desc, rot_dim); F(ta_rope_desc, pos_base);
  Z(ta_rope_desc);
  F(ta_copy_desc, extent); F(ta_copy_desc, src_offset); F(ta_copy_desc, src_strides);
  F(ta_copy_desc, dst_offset); F(ta_copy_desc, dst_strides); Z(ta_copy_desc);
  F(ta_dispatch_info, kernel); F(ta_dispatch_info, tile); F(ta_dispatch_info, has_split_k2);
  F(ta_dispatch_info, split_k2_splits); Z(ta_dispatch_info);
  F(ta_matmul_op_v2, base); F(ta_matmul_op_v2, packed_b); F(ta_matmul_op_v2, reserved); Z(ta_matmul_op_v2);
  F(ta_store_desc, head_dim); F(ta_store_desc, pos_base); F(ta_store_desc, pos_scale);
  F(ta_store_desc, stride_head); F(ta_store_desc, stride_dim); F(ta_store_desc, reserved);
  F(ta_store_desc, pos_addr); Z(ta_store_desc);
  F(ta_matmul_op_v3, v2); F(ta_matmul_op_v3, norm_weight); F(ta_matmul_op_v3, norm_eps);
  F(ta_matmul_op_v3, store_kind); F(ta_matmul_op_v3, store_table); F(ta_matmul_op_v3, store_dst);
  F(ta_matmul_op_v3, store); Z(ta_matmul_op_v3);
  F(ta_flash_desc, kv_len); F(ta_flash_desc, pos_base); F(ta_flash_desc, scale);
  F(ta_flash_desc, token_major_heads); F(ta_flash_desc, out_token_major_heads);
  F(ta_flash_desc, reserved); Z(ta_flash_desc);
  F(ta_rope_scatter_desc, dst_offset); F(ta_rope_scatter_desc, dst_strides);
  F(ta_rope_scatter_desc, pos_scale); F(ta_rope_scatter_desc, reserved); Z(ta_rope_scatter_desc);
  F(ta_prefill_qkv_pack_desc, heads); F(ta_prefill_qkv_pack_desc, kv_heads);
  F(ta_prefill_qkv_pack_desc, head_dim); F(ta_prefill_qkv_pack_desc, rot_dim);
  F(ta_prefill_qkv_pack_desc, pos_base); F(ta_prefill_qkv_pack_desc, reserved);
  Z(ta_prefill_qkv_pack_desc);
  F(ta_attn_decode_desc, kv_len); F(ta_attn_decode_desc, scale); F(ta_attn_decode_desc, pos_addr);
  Z(ta_attn_decode_desc);
  F(ta_exec_op, kind); F(ta_exec_op, mask_kind); F(ta_exec_op, valid_or_prefix);
  F(ta_exec_op, rows_per_group); F(ta_exec_op, scalar); F(ta_exec_op, pos_scale);
  F(ta_exec_op, pos_addr); F(ta_exec_op, in); F(ta_exec_op, out); F(ta_exec_op, matmul);
  F(ta_exec_op, rope); F(ta_exec_op, copy); F(ta_exec_op, flash); F(ta_exec_op, cell);
  F(ta_exec_op, aux); F(ta_exec_op, attn); F(ta_exec_op, aux2); F(ta_exec_op, scatter);
  F(ta_exec_op, binary_op); F(ta_exec_op, qkv); F(ta_exec_op, n_jobs); Z(ta_exec_op);
}

static void die(const char *what) {
  const char *err = ta_last_error();
  fprintf(stderr, "FAIL %s: %s\n", what, err ? err : "(no error text)");
  exit(1);
}

static void expect_close(const char *what, float got, float want, float tol) {
  if (!(fabsf(got - want) <= tol)) {
    fprintf(stderr, "FAIL %s: got %.9g want %.9g\n", what, got, want);
    exit(1);
  }
}

static int run(void) {
  ta_context *ctx = ta_context_create(1, "index:0");
  if (!ctx)
    die("ta_context_create");
  ta_executor *exec = ta_executor_create(ctx, 1, 4, "auto");
  if (!exec)
    die("ta_executor_create");
  const uint32_t sa[2] = {2, 3}, sb[2] = {3, 2}, sc[2] = {2, 2}, sbias[1] = {2};
  ta_tensor *a = ta_tensor_create(ctx, sa, 2), *b = ta_tensor_create(ctx, sb, 2);
  ta_tensor *c = ta_tensor_create(ctx, sc, 2), *bias = ta_tensor_create(ctx, sbias, 1);
  if (!a || !b || !c || !bias)
    die("ta_tensor_create");
  const float ha[6] = {1, 2, 3, 4, 5, 6}, hb[6] = {7, 8, 9, 10, 11, 12}, hbias[2] = {-58.5f, 0.f};
  float hc[4] = {0};
  if (ta_upload(exec, a, ha, 6) || ta_upload(exec, b, hb, 6) || ta_upload(exec, bias, hbias, 2))
    die("ta_upload");

  ta_run_stats st;
  memset(&st, 0, sizeof st);
  if (ta_matmul(exec, a, b, c, 1.0f, 0, &st) || ta_download(exec, c, hc, 4))
    die("ta_matmul");
  const float want[4] = {58, 64, 139, 154};
  for (int i = 0; i < 4; ++i)
    expect_close("plain matmul", hc[i], want[i], 1e-4f);
  if (!st.has_gpu_time || st.n_calls != 1 || st.total_flops != 2 * 2 * 2 * 3)
    die("run stats");
  printf("plain %g %g %g %g flops %llu\n", hc[0], hc[1], hc[2], hc[3],
         (unsigned long long)st.total_flops);

  ta_matmul_op op;
  memset(&op, 0, sizeof op);
  op.call.a = a;
  op.call.b = b;
  op.call.c = c;
  op.call.alpha = 1.0f;
  op.epilogue.bias = bias;
  op.epilogue.activation = TA_ACTIVATION_SILU;
  if (ta_run_ops(exec, &op, 1, &st) || ta_download(exec, c, hc, 4))
    die("ta_run_ops bias+silu");
  const double x = 58.0 - 58.5;
  expect_close("bias+silu c[0]", hc[0], (float)(x / (1.0 + exp(-x))), 1e-5f);
  expect_close("bias+silu c[1]", hc[1], (float)(64.0 / (1.0 + exp(-64.0))), 1e-4f);
  printf("silu %.7g %.7g\n", hc[0], hc[1]);

  ta_prepared *p = ta_prepared_create(exec, &op, 1, 0);
  if (!p)
    die("ta_prepared_create");
  memset(hc, 0, sizeof hc);
  if (ta_upload(exec, c, hc, 4) || ta_prepared_run(p, &st) || ta_prepared_run(p, &st) ||
      ta_download(exec, c, hc, 4))
    die("ta_prepared_run");
  expect_close("prepared c[0]", hc[0], (float)(x / (1.0 + exp(-x))), 1e-5f);
  ta_prepared_destroy(p);

  ta_dispatch_info info;
  if (ta_dispatch_info_for(exec, 1, 2, 2, 3, 0, &info) || !info.kernel)
    die("ta_dispatch_info_for");
  printf("dispatch %s %ux%ux%u\n", info.kernel, info.tile[0], info.tile[1], info.tile[2]);

  ta_tensor_destroy(a);
  ta_tensor_destroy(b);
  ta_tensor_destroy(c);
  ta_tensor_destroy(bias);
  ta_executor_destroy(exec);
  ta_context_destroy(ctx);
  printf("OK\n");
  return 0;
}

int main(int argc, char **argv) {
  if (argc == 2 && strcmp(argv[1], "layout") == 0) {
    layout();
    return 0;
  }
  if (argc == 2 && strcmp(argv[1], "run") == 0)
    return run();
  fprintf(stderr, "usage: %s layout|run\n", argv[0]);
  return 2;
}
