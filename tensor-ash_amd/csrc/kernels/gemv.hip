// Decode GEMV (M = 1..8 rows) for gfx950, HBM-bound, no MFMA.
//
// Replaces the reference's row GEMV family
// (shaders/matmul_row_bda_kernel.glsl:186-403 and the
// matmul_f16w_row_bda_k16{,_v2}{,_packed}.comp wrappers).  Semantics:
// Y[m, :] = epilogue(alpha * X[m, :] @ W (+Y_old)) with f32 accumulation.
// W is f16 (or f32) in either the packed row-tile layout [N/TW][K][TW]
// (src/matmul/api.rs:324-344) or plain row-major [K, N]; both are "tiles
// of TW columns whose rows sit `row_stride` elements apart", so one kernel
// covers both (packed: tile stride K*TW, row stride TW; row-major: tile
// stride TW, row stride N).
//
// Work decomposition: workgroup (256 threads = 4 waves) = one TW-column
// tile x one window of `kchunk` K rows.  A lane owns two adjacent columns
// (one 32-bit f16 pair, or one 64-bit f32 pair), TW/2 lanes span a row,
// so a wave instruction reads 64*4 = 256 contiguous bytes of the packed
// tile.  Each lane issues UNROLL independent loads before its FMAs, giving
// ~32-64 KiB in flight per workgroup.  X for the window sits in LDS as
// [k][MR] so one k costs MR/4 128-bit broadcast reads.
//
// Reduction, fixed order throughout (bit-reproducible):
//   rows of a wave   -> xor shuffles across the 64/(TW/2) row groups;
//   waves            -> LDS, summed wave 0..3;
//   K windows        -> every workgroup stores its partial, the last one
//                       of a tile to arrive (integer counter) sums windows
//                       0..kchunks-1 in order and applies the epilogue.
//
// Dual mode (w2 != null): the same pass reads the two weight matrices of
// a SwiGLU gate/up pair and writes U = alpha * X @ W2 to y2 and
// Y = act(alpha * X @ W + bias) * U to y.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxChunk = 512;
constexpr int kUnroll = 16;

template <int MR, bool DUAL, int TW, bool WF32>
struct Gemv {
  static constexpr int WAYS = DUAL ? 2 : 1;
  static constexpr int LPR = TW / 2;   // lanes per weight row
  static constexpr int RPI = 64 / LPR; // rows per wave instruction
  static constexpr int RPW = RPI * kWaves; // rows per workgroup step
  typedef typename std::conditional<WF32, uint64_t, uint32_t>::type Raw;

  static TA_DEVICE void unpack(Raw raw, float &lo, float &hi) {
    if constexpr (WF32) {
      lo = __builtin_bit_cast(float, (uint32_t)raw);
      hi = __builtin_bit_cast(float, (uint32_t)(raw >> 32));
    } else {
      lo = (float)__builtin_bit_cast(_Float16, (uint16_t)(raw & 0xffffu));
      hi = (float)__builtin_bit_cast(_Float16, (uint16_t)(raw >> 16));
    }
  }

  static TA_DEVICE void run(const GemvArgs &p) {
    __shared__ __attribute__((aligned(16))) float xs[kMaxChunk * MR];
    __shared__ __attribute__((aligned(16))) float red[kWaves * WAYS * MR * TW];
    __shared__ uint32_t last_flag;

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t tiles = (p.n + TW - 1) / TW;
    const uint32_t tile = blockIdx.x % tiles;
    const uint32_t chunk = blockIdx.x / tiles;
    const uint32_t k0 = chunk * p.kchunk;
    const uint32_t kend = min(p.k, k0 + p.kchunk);
    const bool packed = p.flags & TA_GEMV_PACKED;

    // X window -> LDS as [k][MR], zero rows past `rows` and k past kend.
    for (uint32_t i = tid; i < p.kchunk * MR; i += kThreads) {
      const uint32_t kk = i / MR, m = i % MR;
      xs[i] = (m < p.rows && k0 + kk < kend) ? p.x[(uint64_t)m * p.k + k0 + kk] : 0.0f;
    }
    __syncthreads();

    const uint32_t cp = lane % LPR, r0 = lane / LPR;
    const uint32_t col = tile * TW + 2 * cp;
    const bool col_ok = col < p.n; // N % 2 == 0 is required by the host
    const uint64_t tile_base = packed ? (uint64_t)tile * p.k * TW : (uint64_t)tile * TW;
    const uint64_t row_stride = packed ? TW : p.n;
    const Raw *wp[WAYS];
    wp[0] = reinterpret_cast<const Raw *>(
        reinterpret_cast<const char *>(p.w) + (tile_base + 2 * cp) * (WF32 ? 4 : 2));
    if constexpr (DUAL)
      wp[1] = reinterpret_cast<const Raw *>(
          reinterpret_cast<const char *>(p.w2) + (tile_base + 2 * cp) * (WF32 ? 4 : 2));

    float acc[WAYS][MR][2];
#pragma unroll
    for (int w = 0; w < WAYS; ++w)
#pragma unroll
      for (int m = 0; m < MR; ++m)
        acc[w][m][0] = acc[w][m][1] = 0.0f;

    const uint32_t my_first = wave * RPI + r0; // row offset inside a step
    const uint32_t steps = (p.kchunk + RPW - 1) / RPW;
    for (uint32_t s0 = 0; s0 < steps; s0 += kUnroll) {
      Raw raw[WAYS][kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const uint32_t kk = (s0 + u) * RPW + my_first;
        const uint32_t k = k0 + kk;
        const bool ok = col_ok && kk < p.kchunk && k < kend;
#pragma unroll
        for (int w = 0; w < WAYS; ++w)
          raw[w][u] = ok ? *reinterpret_cast<const Raw *>(
                               reinterpret_cast<const char *>(wp[w]) +
                               (uint64_t)k * row_stride * (WF32 ? 4 : 2))
                         : (Raw)0;
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const uint32_t kk = (s0 + u) * RPW + my_first;
        if (kk >= p.kchunk)
          break;
        float xv[MR];
        if constexpr (MR >= 4) {
#pragma unroll
          for (int q = 0; q < MR / 4; ++q) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(&xs[kk * MR + 4 * q]);
            xv[4 * q] = v[0];
            xv[4 * q + 1] = v[1];
            xv[4 * q + 2] = v[2];
            xv[4 * q + 3] = v[3];
          }
        } else {
#pragma unroll
          for (int m = 0; m < MR; ++m)
            xv[m] = xs[kk * MR + m];
        }
#pragma unroll
        for (int w = 0; w < WAYS; ++w) {
          float lo, hi;
          unpack(raw[w][u], lo, hi);
#pragma unroll
          for (int m = 0; m < MR; ++m) {
            acc[w][m][0] = fmaf(xv[m], lo, acc[w][m][0]);
            acc[w][m][1] = fmaf(xv[m], hi, acc[w][m][1]);
          }
        }
      }
    }

    // Rows of one wave: lanes cp, cp + LPR, ... hold the same columns.
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1)
#pragma unroll
      for (int w = 0; w < WAYS; ++w)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          acc[w][m][0] += __shfl_xor(acc[w][m][0], off);
          acc[w][m][1] += __shfl_xor(acc[w][m][1], off);
        }
    if (r0 == 0) {
#pragma unroll
      for (int w = 0; w < WAYS; ++w)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          float *dst = &red[((wave * WAYS + w) * MR + m) * TW + 2 * cp];
          dst[0] = acc[w][m][0];
          dst[1] = acc[w][m][1];
        }
    }
    __syncthreads();

    constexpr int OUTS = WAYS * MR * TW; // this tile's outputs, all ways
    float part[(OUTS + kThreads - 1) / kThreads];
#pragma unroll
    for (int i = 0; i < (OUTS + kThreads - 1) / kThreads; ++i) {
      const uint32_t o = tid + i * kThreads;
      float s = 0.0f;
      if (o < OUTS) {
        s = red[o];
#pragma unroll
        for (int wv = 1; wv < kWaves; ++wv)
          s += red[wv * OUTS + o];
      }
      part[i] = s;
    }

    if (p.kchunks > 1) {
      float *mine = p.partial + ((uint64_t)chunk * tiles + tile) * OUTS;
#pragma unroll
      for (int i = 0; i < (OUTS + kThreads - 1) / kThreads; ++i) {
        const uint32_t o = tid + i * kThreads;
        if (o < OUTS)
          mine[o] = part[i];
      }
      __threadfence();
      __syncthreads();
      if (tid == 0) {
        const uint32_t seen = atomicAdd(&p.counters[tile], 1u);
        last_flag = (seen == p.kchunks - 1) ? 1u : 0u;
      }
      __syncthreads();
      if (!last_flag)
        return;
      __threadfence();
#pragma unroll
      for (int i = 0; i < (OUTS + kThreads - 1) / kThreads; ++i) {
        const uint32_t o = tid + i * kThreads;
        float s = 0.0f;
        if (o < OUTS) {
          const float *src = p.partial + (uint64_t)tile * OUTS + o;
          const uint64_t step = (uint64_t)tiles * OUTS;
          s = __builtin_nontemporal_load(src);
          for (uint32_t c = 1; c < p.kchunks; ++c)
            s += __builtin_nontemporal_load(src + c * step);
        }
        part[i] = s;
      }
      if (tid == 0)
        atomicExch(&p.counters[tile], 0u);
    }

    // Epilogue (shaders/matmul_epilogue_common.glsl:14-21 order).
    if constexpr (DUAL) {
      __syncthreads();
#pragma unroll
      for (int i = 0; i < (OUTS + kThreads - 1) / kThreads; ++i) {
        const uint32_t o = tid + i * kThreads;
        if (o < OUTS)
          red[o] = part[i];
      }
      __syncthreads();
      for (uint32_t o = tid; o < MR * TW; o += kThreads) {
        const uint32_t m = o / TW, c = tile * TW + o % TW;
        if (m >= p.rows || c >= p.n)
          continue;
        const uint64_t yi = (uint64_t)m * p.n + c;
        const float u = p.alpha * red[MR * TW + o];
        float g = p.alpha * red[o];
        if (p.flags & TA_FLAG_BIAS)
          g += p.bias[c];
        p.y2[yi] = u;
        p.y[yi] = ta_activate(g, p.act) * u;
      }
    } else {
#pragma unroll
      for (int i = 0; i < (OUTS + kThreads - 1) / kThreads; ++i) {
        const uint32_t o = tid + i * kThreads;
        const uint32_t m = o / TW, c = tile * TW + o % TW;
        if (o >= OUTS || m >= p.rows || c >= p.n)
          continue;
        const uint64_t yi = (uint64_t)m * p.n + c;
        float v = p.alpha * part[i];
        if (p.flags & TA_FLAG_ACCUMULATE)
          v += p.y[yi];
        if (p.flags & TA_FLAG_BIAS)
          v += p.bias[c];
        v = ta_activate(v, p.act);
        if (p.binary == TA_BIN_ADD_SCALED)
          v = fmaf(p.beta, p.d[yi], v);
        else if (p.binary == TA_BIN_MUL)
          v *= p.d[yi];
        p.y[yi] = v;
      }
    }
  }
};

} // namespace

#define TA_GEMV(NAME, MR, DUAL, TW, WF32)                                          \
  extern "C" __global__ __launch_bounds__(kThreads) void NAME(GemvArgs p) {        \
    Gemv<MR, DUAL, TW, WF32>::run(p);                                              \
  }

#define TA_GEMV_ROWS(PREFIX, DUAL, TW, WF32)                                       \
  TA_GEMV(PREFIX##_m1, 1, DUAL, TW, WF32)                                          \
  TA_GEMV(PREFIX##_m2, 2, DUAL, TW, WF32)                                          \
  TA_GEMV(PREFIX##_m4, 4, DUAL, TW, WF32)                                          \
  TA_GEMV(PREFIX##_m8, 8, DUAL, TW, WF32)

TA_GEMV_ROWS(ta_gemv_f16_t64, false, 64, false)
TA_GEMV_ROWS(ta_gemv_f16_t64_dual, true, 64, false)
TA_GEMV_ROWS(ta_gemv_f16_t32, false, 32, false)
TA_GEMV_ROWS(ta_gemv_f16_t32_dual, true, 32, false)
TA_GEMV_ROWS(ta_gemv_f32_t64, false, 64, true)
