// Device helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernel_args.h"

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

#define TA_DEVICE __device__ __forceinline__

// Activation of the fused epilogue (shaders/matmul_epilogue_common.glsl:
// 30-39 semantics).  The transcendental calls go to the HIP device math
// library; nothing here re-implements them.
TA_DEVICE float ta_activate(float x, uint32_t act) {
  if (act == TA_ACT_RELU)
    return fmaxf(x, 0.0f);
  if (act == TA_ACT_SILU)
    return x / (1.0f + expf(-x));
  if (act == TA_ACT_GELU) {
    // Published tanh form of GELU: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).
    const float k0 = 0.7978845608028654f;
    return 0.5f * x * (1.0f + tanhf(k0 * fmaf(0.044715f * x * x, x, x)));
  }
  return x;
}

// Epilogue order (shaders/matmul_epilogue_common.glsl:14-21):
// v = alpha*acc (+C_old) -> +bias -> act -> (+beta*D | *D).
TA_DEVICE float ta_epilogue(float acc, const GemmArgs &p, uint64_t c_idx,
                            uint32_t col, uint32_t batch) {
  float v = p.alpha * acc;
  if (p.flags & TA_FLAG_ACCUMULATE)
    v += p.c[c_idx];
  if (p.flags & TA_FLAG_BIAS)
    v += p.bias[(uint64_t)batch * p.bias_batch_stride + col];
  v = ta_activate(v, p.act);
  if (p.binary == TA_BIN_ADD_SCALED)
    v = fmaf(p.beta, p.d[c_idx], v);
  else if (p.binary == TA_BIN_MUL)
    v *= p.d[c_idx];
  return v;
}

// XCD-aware tile order.  Workgroups are handed to the 8 XCDs round-robin
// (dispatch id i runs on XCD i % 8), and each XCD has its own L2.  Give
// every XCD a contiguous run of tiles, then walk that run in column groups
// of `group_m` tile rows so neighbouring workgroups on one XCD share A
// row-panels and B column-panels in its L2.
TA_DEVICE void ta_tile_coords(uint32_t lin, uint32_t tiles_m, uint32_t tiles_n,
                              uint32_t &tm, uint32_t &tn) {
  const uint32_t total = tiles_m * tiles_n;
  if ((total & 7u) == 0u) {
    const uint32_t per = total >> 3;
    lin = (lin & 7u) * per + (lin >> 3);
  }
  const uint32_t group_m = 4u;
  const uint32_t in_group = group_m * tiles_n;
  const uint32_t g = lin / in_group;
  const uint32_t first_m = g * group_m;
  const uint32_t rows = min(tiles_m - first_m, group_m);
  const uint32_t r = lin - g * in_group;
  tm = first_m + r % rows;
  tn = r / rows;
}
