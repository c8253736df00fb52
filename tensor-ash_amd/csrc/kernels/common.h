// Device helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "kernel_args.h"

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

#define TA_DEVICE __device__ __forceinline__

// x / y as the hardware reciprocal (v_rcp_f32, about 1 ulp) times x.  The
// IEEE divide sequence the compiler emits for a '/' or __fdividef (scale,
// two Newton steps, fixup) was most of a GELU epilogue's time at one wave
// per SIMD.  y >= 1 wherever it is used here; rcp(inf) = 0.
TA_DEVICE float ta_fast_div(float x, float y) { return x * __builtin_amdgcn_rcpf(y); }

// Activation of the fused epilogue (shaders/matmul_epilogue_common.glsl:
// 30-39 semantics), one instantiation per activation so an epilogue loop
// specialised on it has no per-element branches.  exp is HIP's fast
// __expf (v_exp_f32 on x * log2 e); nothing here re-implements a library
// routine.
template <uint32_t ACT>
TA_DEVICE float ta_act(float x) {
  if constexpr (ACT == TA_ACT_RELU) {
    return fmaxf(x, 0.0f);
  } else if constexpr (ACT == TA_ACT_SILU) {
    return ta_fast_div(x, 1.0f + __expf(-x));
  } else if constexpr (ACT == TA_ACT_GELU) {
    // Published tanh form of GELU, 0.5 x (1 + tanh(u)) with u = sqrt(2/pi)
    // (x + 0.044715 x^3), evaluated through the identity 0.5 (1 + tanh(u))
    // = 1 / (1 + exp(-2u)): one exp and one reciprocal instead of tanh.
    const float k2 = 2.0f * 0.7978845608028654f;
    return ta_fast_div(x, 1.0f + __expf(-k2 * fmaf(0.044715f * x * x, x, x)));
  } else {
    return x;
  }
}

TA_DEVICE float ta_activate(float x, uint32_t act) {
  if (act == TA_ACT_RELU)
    return ta_act<TA_ACT_RELU>(x);
  if (act == TA_ACT_SILU)
    return ta_act<TA_ACT_SILU>(x);
  if (act == TA_ACT_GELU)
    return ta_act<TA_ACT_GELU>(x);
  return x;
}

// Calls f(std::integral_constant<uint32_t, ACT>) for the runtime
// activation, so the loop inside f is compiled once per activation.
template <class F>
TA_DEVICE void ta_with_act(uint32_t act, F &&f) {
  if (act == TA_ACT_RELU)
    f(std::integral_constant<uint32_t, TA_ACT_RELU>{});
  else if (act == TA_ACT_SILU)
    f(std::integral_constant<uint32_t, TA_ACT_SILU>{});
  else if (act == TA_ACT_GELU)
    f(std::integral_constant<uint32_t, TA_ACT_GELU>{});
  else
    f(std::integral_constant<uint32_t, TA_ACT_NONE>{});
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

// Output stage shared by the MFMA GEMMs.  One 32-row block of each wave's
// WTM x WTN sub-tile at a time goes through LDS (the K loop's buffers are
// free after its last barrier): `stage(Cs, blk)` writes block blk of the
// accumulators row-major into the wave's region (row stride WTN + 4), then
// the wave reads it back row-major, applies the epilogue and stores 128-bit
// (f32) or 64-bit (f16) vectors.  This keeps the accumulators in registers
// (no dynamic indexing) and makes the C/D traffic coalesced.
// Split mode (num_splits > 1): alpha * partial to plane (batch*S + split).
// C_F16: C is f16 storage (RNE), only alpha / accumulate apply.
// Waves with `active` false hold no tile and only join the barriers.
template <int WTM, int WTN, int T, bool C_F16, class Stage>
TA_DEVICE void ta_store_tile_staged(float *smem, Stage &&stage, const GemmArgs &p, uint32_t lane,
                                    uint32_t wave, uint32_t wm, uint32_t wn, uint32_t m0,
                                    uint32_t n0, uint32_t batch, uint32_t split,
                                    bool active = true) {
  constexpr int LDC = WTN + 4;
  float *Cs = smem + wave * (32 * LDC);
  const uint32_t S = p.num_splits;
  const uint64_t mn = (uint64_t)p.m * p.n;
  const bool vec_out = (p.n & 3u) == 0u;
#pragma unroll
  for (int fm = 0; fm < WTM / 32; ++fm) {
    if (active)
      stage(Cs, fm);
    __syncthreads();
    const uint32_t row0 = m0 + wm * WTM + fm * 32;
    const uint32_t col0 = n0 + wn * WTN;
    // A lane's column quad is the same on every row it stores (64 lanes
    // step through rows of WTN / 4 quads), so its bias quad is loaded once
    // per block, not once per row: inside the loop each load's latency
    // stood between the LDS read and the store.
    static_assert(64 % (WTN / 4) == 0, "a lane keeps its columns across rows");
    f32x4 bias_q = {0.f, 0.f, 0.f, 0.f};
    if (!C_F16 && S == 1 && active && (p.flags & TA_FLAG_BIAS) && vec_out) {
      const uint32_t col = col0 + (lane % (WTN / 4)) * 4;
      if (col + 4 <= p.n)
        bias_q = *reinterpret_cast<const f32x4 *>(
            &p.bias[(uint64_t)batch * p.bias_batch_stride + col]);
    }
    ta_with_act(S > 1 ? (uint32_t)TA_ACT_NONE : p.act, [&](auto act_c) __attribute__((always_inline)) {
    constexpr uint32_t ACT = decltype(act_c)::value;
#pragma unroll 2
    for (int i = 0; i < (active ? 32 * WTN / 4 / 64 : 0); ++i) {
      const uint32_t e = lane + 64u * i;
      const uint32_t lrow = e / (WTN / 4), c4 = (e % (WTN / 4)) * 4;
      const uint32_t row = row0 + lrow, col = col0 + c4;
      if (row >= p.m || col >= p.n)
        continue;
      const f32x4 v = *reinterpret_cast<const f32x4 *>(&Cs[lrow * LDC + c4]);
      const uint64_t base = S > 1 ? ((uint64_t)batch * S + split) * mn + (uint64_t)row * p.n + col
                                  : (uint64_t)batch * p.stride_c + (uint64_t)row * p.n + col;
      if constexpr (C_F16) {
        _Float16 *c16 = reinterpret_cast<_Float16 *>(p.c);
        const bool acc_old = p.flags & TA_FLAG_ACCUMULATE;
        if (vec_out && col + 4 <= p.n) {
          f16x4 old = acc_old ? *reinterpret_cast<const f16x4 *>(c16 + base) : f16x4{0, 0, 0, 0};
          f16x4 o;
#pragma unroll
          for (int c = 0; c < 4; ++c)
            o[c] = (_Float16)(p.alpha * v[c] + (acc_old ? (float)old[c] : 0.0f));
          *reinterpret_cast<f16x4 *>(c16 + base) = o;
        } else {
          for (int c = 0; c < 4 && col + c < p.n; ++c)
            c16[base + c] =
                (_Float16)(p.alpha * v[c] + (acc_old ? (float)c16[base + c] : 0.0f));
        }
      } else if (vec_out && col + 4 <= p.n) {
        // ta_epilogue on four columns with 128-bit loads of C, bias and D.
        f32x4 o = p.alpha * v;
        if (S == 1) {
          if (p.flags & TA_FLAG_ACCUMULATE)
            o += *reinterpret_cast<const f32x4 *>(&p.c[base]);
          if (p.flags & TA_FLAG_BIAS)
            o += bias_q;
#pragma unroll
          for (int c = 0; c < 4; ++c)
            o[c] = ta_act<ACT>(o[c]);
          if (p.binary != TA_BIN_NONE) {
            const f32x4 d = *reinterpret_cast<const f32x4 *>(&p.d[base]);
#pragma unroll
            for (int c = 0; c < 4; ++c)
              o[c] = p.binary == TA_BIN_ADD_SCALED ? fmaf(p.beta, d[c], o[c]) : o[c] * d[c];
          }
        }
        *reinterpret_cast<f32x4 *>(&p.c[base]) = o;
        if (p.c16) {
          f16x4 h;
#pragma unroll
          for (int c = 0; c < 4; ++c)
            h[c] = (_Float16)o[c];
          *reinterpret_cast<f16x4 *>(reinterpret_cast<_Float16 *>(p.c16) + base) = h;
        }
      } else {
        for (int c = 0; c < 4 && col + c < p.n; ++c) {
          const float r = S > 1 ? p.alpha * v[c] : ta_epilogue(v[c], p, base + c, col + c, batch);
          p.c[base + c] = r;
          if (p.c16)
            reinterpret_cast<_Float16 *>(p.c16)[base + c] = (_Float16)r;
        }
      }
    }
    });
    __syncthreads();
  }
}

// ta_store_tile_staged for the 32x32 MFMA accumulator layout: lane l,
// register r holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
template <int WTM, int WTN, int FM, int FN, int T, bool C_F16>
TA_DEVICE void ta_store_tile(float *smem, int smem_floats, const f32x16 (&acc)[FM][FN],
                             const GemmArgs &p, uint32_t lane, uint32_t wave, uint32_t wm,
                             uint32_t wn, uint32_t m0, uint32_t n0, uint32_t batch,
                             uint32_t split, bool active = true) {
  (void)smem_floats;
  constexpr int LDC = WTN + 4;
  const uint32_t lr = lane & 31u, lg = lane >> 5;
  auto stage = [&](float *Cs, int fm) __attribute__((always_inline)) {
#pragma unroll
    for (int f = 0; f < FM; ++f) {
      if (f != fm)
        continue;
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          Cs[(8 * (r / 4) + 4 * lg + (r % 4)) * LDC + fn * 32 + lr] = acc[f][fn][r];
    }
  };
  ta_store_tile_staged<WTM, WTN, T, C_F16>(smem, stage, p, lane, wave, wm, wn, m0, n0, batch,
                                           split, active);
}
