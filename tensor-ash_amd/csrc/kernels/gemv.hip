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
// tile x one window of `kchunk` K rows.  A lane owns CPL adjacent columns
// read with one 64-bit load (four f16 or two f32), TW/CPL lanes span a
// row, so one wave instruction reads 512 contiguous bytes of the packed
// tile.  Each lane issues all kUnroll loads of a group unconditionally
// (rows past the window re-read a valid row and are zeroed afterwards) so
// they are in flight together.  X for the window sits in LDS as [k][MR]
// so one k costs MR/4 128-bit broadcast reads.
//
// Reduction, fixed order throughout (bit-reproducible):
//   rows of a wave   -> xor shuffles across the 64/(TW/CPL) row groups;
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

template <int MR, bool DUAL, int TW, bool WF32>
struct Gemv {
  static constexpr int WAYS = DUAL ? 2 : 1;
  static constexpr int kMaxChunk = 4096 / MR; // X-window rows held in LDS (16 KiB)
  static constexpr int CPL = WF32 ? 2 : 4;   // columns per lane (8-byte load)
  static constexpr int LPR = TW / CPL;       // lanes per weight row
  static constexpr int RPI = 64 / LPR;       // rows per wave instruction
  static constexpr int RPW = RPI * kWaves;   // rows per workgroup step
  static constexpr int EB = WF32 ? 4 : 2;    // bytes per weight element
  static constexpr int kUnroll = 16; // loads per weight matrix per group

  static TA_DEVICE void unpack(uint64_t raw, float (&v)[CPL]) {
    if constexpr (WF32) {
      v[0] = __builtin_bit_cast(float, (uint32_t)raw);
      v[1] = __builtin_bit_cast(float, (uint32_t)(raw >> 32));
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        v[c] = (float)__builtin_bit_cast(_Float16, (uint16_t)(raw >> (16 * c)));
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

    const uint32_t cp = lane % LPR, r0 = lane / LPR;
    // Lanes past N (row-major, ragged last tile) read column 0 of the tile
    // and have their values discarded: every load below is unconditional,
    // so the compiler keeps all of a group's loads in flight.
    const uint32_t col = tile * TW + CPL * cp;
    const bool col_ok = col + CPL <= p.n; // host requires N % CPL == 0
    const uint64_t tile_base = packed ? (uint64_t)tile * p.k * TW : (uint64_t)tile * TW;
    const uint64_t row_stride = (packed ? TW : p.n) * (uint64_t)EB;
    const uint64_t lane_off = (tile_base + (col_ok ? CPL * cp : 0)) * EB;
    const char *wp[WAYS];
    wp[0] = reinterpret_cast<const char *>(p.w) + lane_off;
    if constexpr (DUAL)
      wp[1] = reinterpret_cast<const char *>(p.w2) + lane_off;
    const uint32_t my_first = wave * RPI + r0;
    constexpr uint32_t G = RPW * kUnroll; // rows per unrolled group

    // One group of loads; rows at or past kend re-read row k0 (valid, and
    // zeroed before use), so the loads carry no branches.
    auto issue = [&](uint32_t kb, uint64_t (&raw)[WAYS][kUnroll]) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const uint32_t k = k0 + kb + u * RPW + my_first;
        const uint32_t kc = k < kend ? k : k0;
#pragma unroll
        for (int w = 0; w < WAYS; ++w)
          raw[w][u] = __builtin_nontemporal_load(
              reinterpret_cast<const uint64_t *>(wp[w] + (uint64_t)kc * row_stride));
      }
    };

    // X loads go out first, then the first weight group: vmcnt retires in
    // issue order, so staging X into LDS then waits only for X.
    constexpr int XPT = kMaxChunk * MR / kThreads;
    float xr[XPT];
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
      const uint32_t i = tid + j * kThreads;
      const uint32_t kk = i / MR, m = i % MR;
      const bool ok = i < p.kchunk * MR && m < p.rows && k0 + kk < kend;
      xr[j] = p.x[ok ? (uint64_t)m * p.k + k0 + kk : 0];
      xr[j] = ok ? xr[j] : 0.0f;
    }
    uint64_t cur[WAYS][kUnroll];
    issue(0, cur);
#pragma unroll
    for (int j = 0; j < XPT; ++j)
      xs[tid + j * kThreads] = xr[j];
    __syncthreads();

    float acc[WAYS][MR][CPL];
#pragma unroll
    for (int w = 0; w < WAYS; ++w)
#pragma unroll
      for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int c = 0; c < CPL; ++c)
          acc[w][m][c] = 0.0f;

    auto consume = [&](uint32_t kb, const uint64_t (&raw)[WAYS][kUnroll]) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const uint32_t kk = kb + u * RPW + my_first;
        const bool ok = k0 + kk < kend && col_ok;
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
          float wv[CPL];
          unpack(ok ? raw[w][u] : 0ull, wv);
#pragma unroll
          for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int c = 0; c < CPL; ++c)
              acc[w][m][c] = fmaf(xv[m], wv[c], acc[w][m][c]);
        }
      }
    };

    // kchunk is a multiple of G (host contract): whole groups only.  The
    // resident grid (every workgroup of a decode launch fits at once)
    // keeps HBM busy while each wave waits on its own group.
    consume(0, cur);
    for (uint32_t kb = G; kb < p.kchunk; kb += G) {
      issue(kb, cur);
      consume(kb, cur);
    }

    // Rows of one wave: lanes cp, cp + LPR, ... hold the same columns.
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1)
#pragma unroll
      for (int w = 0; w < WAYS; ++w)
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
          for (int c = 0; c < CPL; ++c)
            acc[w][m][c] += __shfl_xor(acc[w][m][c], off);
    if (r0 == 0) {
#pragma unroll
      for (int w = 0; w < WAYS; ++w)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          float *dst = &red[((wave * WAYS + w) * MR + m) * TW + CPL * cp];
#pragma unroll
          for (int c = 0; c < CPL; ++c)
            dst[c] = acc[w][m][c];
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
      // Cross-XCD hand-off without an L2 write-back: partials are written
      // and read only with agent-scope relaxed atomics (sc1 loads/stores,
      // coherent per location across the XCDs' L2s).  Waiting for this
      // thread's stores to complete before the barrier makes them visible
      // before thread 0 bumps the tile counter (release); the last
      // workgroup reads them after observing the count (acquire by control
      // dependency).  __threadfence() would instead write back and
      // invalidate the whole L2 in every workgroup.
      float *mine = p.partial + ((uint64_t)chunk * tiles + tile) * OUTS;
#pragma unroll
      for (int i = 0; i < (OUTS + kThreads - 1) / kThreads; ++i) {
        const uint32_t o = tid + i * kThreads;
        if (o < OUTS)
          __hip_atomic_store(mine + o, part[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (tid == 0) {
        const uint32_t seen =
            __hip_atomic_fetch_add(&p.counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_flag = (seen == p.kchunks - 1) ? 1u : 0u;
      }
      __syncthreads();
      if (!last_flag)
        return;
      // Sum the windows in order 0..kchunks-1.  All partial loads of a
      // batch go out at once (one memory round trip) into the X window's
      // LDS, which is free now; then each output is summed sequentially.
      const uint64_t step = (uint64_t)tiles * OUTS;
      const float *tsrc = p.partial + (uint64_t)tile * OUTS;
      constexpr uint32_t NB = (kMaxChunk * MR) / OUTS; // windows per batch
      float sum[(OUTS + kThreads - 1) / kThreads];
#pragma unroll
      for (int i = 0; i < (OUTS + kThreads - 1) / kThreads; ++i)
        sum[i] = 0.0f;
      for (uint32_t c0 = 0; c0 < p.kchunks; c0 += NB) {
        const uint32_t nb = min(NB, p.kchunks - c0);
        __syncthreads(); // previous batch fully consumed
        for (uint32_t e = tid; e < nb * OUTS; e += kThreads) {
          const uint32_t c = c0 + e / OUTS, o = e % OUTS;
          xs[e] = __hip_atomic_load(tsrc + c * step + o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < (OUTS + kThreads - 1) / kThreads; ++i) {
          const uint32_t o = tid + i * kThreads;
          if (o < OUTS)
            for (uint32_t c = 0; c < nb; ++c)
              sum[i] = (c0 + c == 0) ? xs[o] : sum[i] + xs[c * OUTS + o];
        }
      }
#pragma unroll
      for (int i = 0; i < (OUTS + kThreads - 1) / kThreads; ++i)
        part[i] = sum[i];
      if (tid == 0)
        __hip_atomic_store(&p.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
