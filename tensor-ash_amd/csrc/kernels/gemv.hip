// Decode GEMV (M = 1..8 rows) for gfx950, HBM-bound, and the persistent
// decode SwiGLU MLP built from it.  1-2 rows and f32 or 32-column weights
// use vector FMAs; f16 64-column tiles with 4-8 rows use f16 MFMAs on X
// split into three f16 pieces (Gemv::stage_split).
//
// Replaces the reference's row GEMV family
// (shaders/matmul_row_bda_kernel.glsl:186-403 and the
// matmul_f16w_row_bda_k16{,_v2}{,_packed}.comp wrappers) and plays the
// role of its persistent GEMV chain (shaders/matmul_gemv_chain_kernel.glsl)
// for the decode MLP.  Semantics: Y[m, :] = epilogue(alpha * X[m, :] @ W
// (+Y_old)) with f32 accumulation.  W is f16 (or f32) in either the packed
// row-tile layout [N/TW][K][TW] (src/matmul/api.rs:324-344) or plain
// row-major [K, N]; both are "tiles of TW columns whose rows sit
// `row_stride` elements apart", so one kernel covers both (packed: tile
// stride K*TW, row stride TW; row-major: tile stride TW, row stride N).
//
// Work unit: 256 threads (4 waves) = one TW-column tile x one window of
// `kchunk` K rows.  A lane owns CPL adjacent columns read with one 64-bit
// load (four f16 or two f32), TW/CPL lanes span a row, so one wave
// instruction reads 512 contiguous bytes of the packed tile.  Each lane
// issues all kUnroll loads of a group unconditionally (rows past the window
// re-read a valid row and are zeroed afterwards) so they are in flight
// together.  X for the window sits in LDS as [k][MR] so one k costs MR/4
// 128-bit broadcast reads.
//
// Reduction, fixed order throughout (bit-reproducible):
//   rows of a wave   -> xor shuffles across the 64/(TW/CPL) row groups;
//   waves            -> LDS, summed wave 0..3;
//   K windows        -> every unit stores its partial, the last one of a
//                       tile to arrive (integer counter) sums windows
//                       0..kchunks-1 in order and applies the epilogue.
// The cross-workgroup hand-off uses agent-scope relaxed atomics only
// (sc1 loads/stores, coherent per location across the XCDs' L2s); a
// vmcnt(0) wait before the barrier orders the partial stores before the
// counter increment.  __threadfence() would write back and invalidate the
// whole L2 in every workgroup.
//
// Dual mode (w2 != null): the same pass reads the two weight matrices of
// a SwiGLU gate/up pair and writes U = alpha * X @ W2 to y2 and
// Y = act(alpha * X @ W + bias) * U to y.
#include "common.h"

// Row counts from which the matrix-core route and the hand-off sentinel
// pre-poll apply (compile-time, for measurement builds).
#ifndef TA_GEMV_MFMA_MIN_ROWS
#define TA_GEMV_MFMA_MIN_ROWS 4
#endif
#ifndef TA_GEMV_SENTINEL_MIN_ROWS
#define TA_GEMV_SENTINEL_MIN_ROWS 4
#endif
#ifndef TA_MLP_ISSUE_BATCH_M1
#define TA_MLP_ISSUE_BATCH_M1 2
#endif
#ifndef TA_MLP_ISSUE_BATCH_M2
#define TA_MLP_ISSUE_BATCH_M2 2
#endif
#ifndef TA_MLP_ISSUE_BATCH_M4
#define TA_MLP_ISSUE_BATCH_M4 0
#endif
#ifndef TA_MLP_ISSUE_BATCH_M8
#define TA_MLP_ISSUE_BATCH_M8 2
#endif

namespace {

constexpr int kThreads = 256;
// Row values of a normed-A GEMV at one row loaded per thread ahead of the
// weight stream (the rest of a longer row is read after it).
constexpr int kNormPre = 8;
constexpr int kWaves = kThreads / 64;

// Standalone launch, decode-MLP producer (gate/up, publishes tagged h),
// decode-MLP consumer (down-proj, polls the tagged h its window reads).
enum { kStandalone = 0, kProducer = 1, kConsumer = 2 };

TA_DEVICE float coherent_load(const float *p) {
  return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
TA_DEVICE void coherent_store(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A workgroup-uniform pointer, moved to scalar registers so a load can use
// it as its scalar base with a 32-bit per-lane offset.
typedef __attribute__((address_space(1))) const char global_char;
TA_DEVICE global_char *uniform_ptr(const char *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<global_char *>(((uint64_t)hi << 32) | lo);
}

// Decode-MLP hand-off word: f32 value bits low, launch tag high; one
// naturally aligned 64-bit access, so a reader sees value and tag together.
TA_DEVICE uint64_t tag_word(float v, uint32_t tag) {
  return ((uint64_t)tag << 32) | __builtin_bit_cast(uint32_t, v);
}
TA_DEVICE uint64_t load_word(const uint64_t *p) {
  return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
TA_DEVICE void store_word(uint64_t *p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every thread reads N tagged words (address at(j), needed when need(j));
// the workgroup re-reads them all until every needed word of every thread
// carries `tag`, sleeping ~0.05 us between rounds.  out[] holds the values
// of the last round.  Bounded: after spin_limit rounds in all (`polls`
// counts rounds a pre-poll already spent) the wait gives up and raises the
// host-visible status word (the launch's results are then invalid).
template <int N, class At, class Need>
TA_DEVICE void poll_words(At at, Need need, uint32_t tag, float (&out)[N], const MlpArgs &m,
                          uint32_t polls = 0) {
  for (;;) {
    uint64_t w[N];
#pragma unroll
    for (int j = 0; j < N; ++j)
      w[j] = load_word(at(j));
    int ok = 1;
#pragma unroll
    for (int j = 0; j < N; ++j) {
      ok &= (!need(j) || (uint32_t)(w[j] >> 32) == tag) ? 1 : 0;
      out[j] = __builtin_bit_cast(float, (uint32_t)w[j]);
    }
    if (__syncthreads_and(ok))
      return;
    if (++polls >= m.spin_limit) {
      if (threadIdx.x == 0)
        __hip_atomic_store(m.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      return;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// Decode-MLP hand-off pre-poll.  Before reading a window's published
// words [col][MR] (a whole round of loads per thread, repeated until all
// carry the tag), wait on one sentinel word per producer tile -- its
// column 63 at row `row` (the last row written) -- with 4 or 8 loads a
// round from wave 0.  The tile's stores go out together, so the rest have
// nearly always landed by then; the window's words are then read and
// their tags checked as before (poll_words), so a sentinel seen early
// costs another round, never a wrong value.  Used from M = 4 up: with
// fewer rows the window's words are few enough that the extra round trip
// costs more than the re-reads it saves.  Returns the rounds it spent, which
// the word poll that follows counts against the same spin_limit (so a lost
// hand-off is reported after one bound, not two).
TA_DEVICE uint32_t poll_sentinels(const uint64_t *words, uint32_t first_tile, uint32_t ntiles,
                                  uint32_t mr, uint32_t row, uint32_t tag, const MlpArgs &m) {
  const uint32_t tid = threadIdx.x;
  const uint64_t *f = words + ((uint64_t)(first_tile + tid) * 64u + 63u) * mr + row;
  for (uint32_t polls = 0;;) {
    const bool ok = tid >= ntiles || (uint32_t)(load_word(f) >> 32) == tag;
    if (__syncthreads_and(ok))
      return polls;
    if (++polls >= m.spin_limit)
      return polls - 1u; // the word poll still takes its one round
    __builtin_amdgcn_s_sleep(2);
  }
}

// COH (persistent GEMV chain): X, the normed-A row and D are read, and Y
// is written, with agent-scope accesses, so a job may read what an earlier
// job of the same launch wrote on another XCD once a grid barrier (no
// cache-wide fences) has passed.
template <int MR, bool DUAL, int TW, bool WF32, int MODE, int XROWS, int UNROLL = 16,
          bool COH = false>
struct Gemv {
  static constexpr int WAYS = DUAL ? 2 : 1;
  static constexpr int CPL = WF32 ? 2 : 4;  // columns per lane (8-byte load)
  static constexpr int LPR = TW / CPL;      // lanes per weight row
  static constexpr int RPI = 64 / LPR;      // rows per wave instruction
  static constexpr int RPW = RPI * kWaves;  // rows per workgroup step
  static constexpr int EB = WF32 ? 4 : 2;   // bytes per weight element
  static constexpr int kUnroll = UNROLL;    // loads per weight matrix per group
  // Decode-MLP units: weight loads per issue batch (at most two batches
  // outstanding while the window is fetched; 0 = all at once).
  static constexpr int kIssueBatch = MR == 1   ? TA_MLP_ISSUE_BATCH_M1
                                     : MR == 2 ? TA_MLP_ISSUE_BATCH_M2
                                     : MR == 4 ? TA_MLP_ISSUE_BATCH_M4
                                               : TA_MLP_ISSUE_BATCH_M8;
  static constexpr int OUTS = WAYS * MR * TW; // outputs of one tile, all ways
  static constexpr int OPT = (OUTS + kThreads - 1) / kThreads;
  // The X window's LDS is reused to stage the partials of all K windows
  // for the last unit of a tile: PSTAGE floats, 16 loads per thread.
  static constexpr int PSTAGE = 16 * kThreads;
  // Decode-MLP tile reducers poll the other windows' words in rounds of
  // MPOLL loads per thread: each further round is another poll round trip
  // behind the weight stream.  One round covers the 7 (gate/up) or 10
  // (down) other windows of the 2048 x 5632 layer up to M = 4; M = 8 takes
  // two (32 loads a round spill).
  static constexpr int MPOLL = MODE == kStandalone || MR == 1 ? 8 : 16;
  static constexpr int PST = PSTAGE > MPOLL * kThreads ? PSTAGE : MPOLL * kThreads;
  static constexpr int XS0 = XROWS * MR > PST ? XROWS * MR : PST;
  // Matrix-core route (f16 weights, 64-column tiles, 4..8 rows): each weight
  // would otherwise feed MR vector FMAs, which at M >= 4 outlast the weight
  // stream once X has arrived.  X is staged as three f16 pieces per value
  // (3 * XROWS * MR halfs) instead of f32.
  static constexpr bool MF = !WF32 && TW == 64 && MR >= TA_GEMV_MFMA_MIN_ROWS;
  static constexpr int XSMF = MF ? (3 * XROWS * MR + 1) / 2 : 0;
  static constexpr int XS = XS0 > XSMF ? XS0 : XSMF;

  struct Smem {
    float xs[XS]; // X window, later the partials of the last unit
    float red[kWaves * OUTS];
    float xmax[kWaves * 8]; // matrix-core route: per-wave row maxima
    float xinv[8];          // and the rows' inverse scales
    uint32_t last_flag;
  };

  static TA_DEVICE void unpack(uint64_t raw, float (&v)[CPL]) {
    if constexpr (WF32) {
      v[0] = __builtin_bit_cast(float, (uint32_t)raw);
      v[1] = __builtin_bit_cast(float, (uint32_t)(raw >> 32));
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v[c] = (float)__builtin_bit_cast(_Float16, (uint16_t)(raw >> (16 * c)));
        // Keep the widening a separate v_cvt_f32_f16: folded into every
        // FMA it becomes v_fma_mix_f32, which issues at half the rate of
        // v_fma_f32 on gfx950, and each weight feeds MR FMAs.
        if constexpr (MR > 1)
          asm volatile("" : "+v"(v[c]));
      }
    }
  }

  static TA_DEVICE void unit(const GemvArgs &p, uint32_t tile, uint32_t chunk, Smem &sm,
                             const MlpArgs *mlp = nullptr, uint32_t layer = 0,
                             const GemvFusion *fu = nullptr) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t tiles = (p.n + TW - 1) / TW;
    const uint32_t k0 = chunk * p.kchunk;
    const uint32_t kend = min(p.k, k0 + p.kchunk);
    const bool packed = p.flags & TA_GEMV_PACKED;
    // Decode MLP: this layer's hand-off tag (read before any hand-off).
    uint32_t tag = 0;
    if constexpr (MODE != kStandalone)
      tag = __hip_atomic_load(mlp->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + layer + 1u;

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

    // Decode-MLP units cover whole packed tiles and whole K windows (host
    // contract), so no row or column is ragged: the loads address a
    // uniform row base plus one per-lane 32-bit offset (scalar-base loads,
    // one address register), and no value needs masking.
    constexpr bool EXACT = MODE != kStandalone;
    const char *wbase[WAYS];
    wbase[0] = reinterpret_cast<const char *>(p.w) + tile_base * EB;
    if constexpr (DUAL)
      wbase[1] = reinterpret_cast<const char *>(p.w2) + tile_base * EB;
    const uint32_t lane_b = my_first * (uint32_t)row_stride + CPL * cp * EB;

    // One group of loads; rows at or past kend re-read row k0 (valid, and
    // zeroed before use), so the loads carry no branches.
    auto issue = [&](uint32_t kb, uint64_t (&raw)[WAYS][kUnroll]) {
      if constexpr (EXACT) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
          for (int w = 0; w < WAYS; ++w)
            raw[w][u] = __builtin_nontemporal_load(
                reinterpret_cast<__attribute__((address_space(1))) const uint64_t *>(
                    uniform_ptr(wbase[w] + (uint64_t)(k0 + kb + u * RPW) * row_stride) + lane_b));
          // Decode-MLP units keep at most 2 * kIssueBatch of their loads
          // outstanding: every resident unit fetching its whole window at
          // once queues ~64 MB at the memory controllers, and each hand-off
          // poll then waits behind that queue.  The window still lands in
          // registers long before the unit's input is published.
          const int issued = (u + 1) * WAYS;
          if (kIssueBatch > 0 && issued % kIssueBatch == 0 && issued >= 2 * kIssueBatch &&
              issued < kUnroll * WAYS)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kIssueBatch) : "memory");
        }
        return;
      }
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

    // X window: XPT values per thread, clamped index + select (no branch).
    constexpr int XPT = XROWS * MR / kThreads;
    float xr[XPT];
    auto x_index = [&](int j, bool &ok) {
      const uint32_t i = tid + j * kThreads;
      const uint32_t kk = i / MR, m = i % MR;
      ok = i < p.kchunk * MR && m < p.rows && k0 + kk < kend;
      return ok ? (uint64_t)m * p.k + k0 + kk : 0;
    };

    uint64_t cur[WAYS][kUnroll];
    if constexpr (MODE == kConsumer) {
      // Weights first (they do not depend on X), then poll the tagged h
      // words of the window ([k][MR] order) until all carry this launch's
      // tag; vmcnt retires in order, so the first poll lands after them.
      issue(0, cur);
      uint32_t spent = 0;
      if constexpr (MR >= TA_GEMV_SENTINEL_MIN_ROWS)
        spent = poll_sentinels(mlp->tag_h, k0 / 64u, (kend - k0) / 64u, MR, p.rows - 1u, tag,
                               *mlp);
      poll_words<XPT>(
          [&](int j) {
            bool ok;
            (void)x_index(j, ok);
            const uint32_t i = tid + j * kThreads;
            return mlp->tag_h + (ok ? (uint64_t)k0 * MR + i : 0);
          },
          [&](int j) {
            bool ok;
            (void)x_index(j, ok);
            return ok;
          },
          tag, xr, *mlp, spent);
#pragma unroll
      for (int j = 0; j < XPT; ++j) {
        bool ok;
        (void)x_index(j, ok);
        xr[j] = ok ? xr[j] : 0.0f;
      }
    } else if (MODE == kProducer && layer > 0) {
      // Chained layer: weights first, then X = the previous layer's y from
      // its tagged words ([k][MR] order, the previous layer's tag).
      issue(0, cur);
      uint32_t spent = 0;
      if constexpr (MR >= TA_GEMV_SENTINEL_MIN_ROWS)
        spent = poll_sentinels(mlp->tag_y, k0 / 64u, (kend - k0) / 64u, MR, p.rows - 1u, tag - 1u,
                               *mlp);
      poll_words<XPT>(
          [&](int j) {
            bool ok;
            (void)x_index(j, ok);
            const uint32_t i = tid + j * kThreads;
            return mlp->tag_y + (ok ? (uint64_t)k0 * MR + i : 0);
          },
          [&](int j) {
            bool ok;
            (void)x_index(j, ok);
            return ok;
          },
          tag - 1u, xr, *mlp, spent);
#pragma unroll
      for (int j = 0; j < XPT; ++j) {
        bool ok;
        (void)x_index(j, ok);
        xr[j] = ok ? xr[j] : 0.0f;
      }
    } else {
      // X loads go out first, then the first weight group: vmcnt retires
      // in issue order, so staging X into LDS then waits only for X.  With
      // normed A at one row, the row's first kNormPre * kThreads values
      // (its sum of squares) are loaded before the weights too, so the
      // norm does not wait behind the weight stream.
#pragma unroll
      for (int j = 0; j < XPT; ++j) {
        bool ok;
        const uint64_t xi = x_index(j, ok);
        xr[j] = COH ? coherent_load(p.x + xi) : p.x[xi];
        xr[j] = ok ? xr[j] : 0.0f;
      }
      // Normed A: the standalone launch's fusion, or the first layer of a
      // decode MLP (its x is read from memory, like a standalone launch's).
      const float *norm_w = nullptr;
      float norm_eps = 0.0f;
      if constexpr (MODE == kStandalone) {
        if (fu && fu->norm_w) {
          norm_w = fu->norm_w;
          norm_eps = fu->norm_eps;
        }
      } else if constexpr (MODE == kProducer) {
        norm_w = mlp->norm_w;
        norm_eps = mlp->norm_eps;
      }
      float pre[kNormPre];
      if constexpr (MODE != kConsumer && MR == 1) {
        if (norm_w) {
#pragma unroll
          for (int i = 0; i < kNormPre; ++i) {
            const uint32_t kk = tid + i * kThreads;
            const uint32_t at = min(kk, p.k - 1u);
            const float v = COH ? coherent_load(p.x + at) : p.x[at];
            pre[i] = kk < p.k ? v : 0.0f;
          }
        }
      }
      issue(0, cur);
      if constexpr (MODE != kConsumer) {
        if (norm_w)
          normalize_x(p, norm_w, norm_eps, k0, xr, sm, pre);
      }
    }
    if constexpr (MF) {
      stage_split(xr, sm);
    } else {
#pragma unroll
      for (int j = 0; j < XPT; ++j)
        sm.xs[tid + j * kThreads] = xr[j];
    }
    __syncthreads();

    float acc[WAYS][MR][CPL];
#pragma unroll
    for (int w = 0; w < WAYS; ++w)
#pragma unroll
      for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int c = 0; c < CPL; ++c)
          acc[w][m][c] = 0.0f;

    // X rows are read from LDS in batches of XB (8 floats), all reads of
    // a batch before any use, so their latencies overlap.
    constexpr int XB = MR >= 8 ? 1 : 8 / MR;
    static_assert(kUnroll % XB == 0, "whole X batches per group");
    auto consume = [&](uint32_t kb, const uint64_t (&raw)[WAYS][kUnroll]) {
#pragma unroll
      for (int u0 = 0; u0 < kUnroll; u0 += XB) {
        float xv[XB][MR];
#pragma unroll
        for (int b = 0; b < XB; ++b) {
          const uint32_t kk = kb + (u0 + b) * RPW + my_first;
          if constexpr (MR >= 4) {
#pragma unroll
            for (int q = 0; q < MR / 4; ++q) {
              const f32x4 v = *reinterpret_cast<const f32x4 *>(&sm.xs[kk * MR + 4 * q]);
              xv[b][4 * q] = v[0];
              xv[b][4 * q + 1] = v[1];
              xv[b][4 * q + 2] = v[2];
              xv[b][4 * q + 3] = v[3];
            }
          } else {
#pragma unroll
            for (int m = 0; m < MR; ++m)
              xv[b][m] = sm.xs[kk * MR + m];
          }
        }
#pragma unroll
        for (int b = 0; b < XB; ++b) {
          const int u = u0 + b;
          const uint32_t kk = kb + u * RPW + my_first;
          const bool ok = EXACT || (k0 + kk < kend && col_ok);
#pragma unroll
          for (int w = 0; w < WAYS; ++w) {
            float wv[CPL];
            unpack(ok ? raw[w][u] : 0ull, wv);
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
              for (int c = 0; c < CPL; ++c)
                acc[w][m][c] = fmaf(xv[b][m], wv[c], acc[w][m][c]);
          }
        }
      }
    };

    // Matrix-core route.  v_mfma_f32_16x16x16_f16 computes D[m][n] +=
    // sum_k A[m][k] B[k][n] with lane l holding A[l%16][4(l/16)+i],
    // B[4(l/16)+i][l%16] and D[4(l/16)+i][l%16], i = 0..3.  A lane's loads
    // 4j..4j+3 of a group hold 4 rows x its 4 columns 4cp..4cp+3 (cp =
    // l%16, row group r0 = l/16), so byte permutes inside the lane give
    // block c's B operand (those 4 rows of column 4cp+c): k slot 4*r0 + i
    // is window row kb + 64j + 16i + 4*wave + r0, for every block.  A is
    // X's three pieces at the same rows (rows m >= MR duplicate row m % MR;
    // their outputs are dropped).  Passes hi, mid, lo per step, blocks
    // interleaved so consecutive MFMAs are independent.
    f32x4 macc[WAYS][4];
#pragma unroll
    for (int w = 0; w < WAYS; ++w)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        macc[w][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto consume_mf = [&](uint32_t kb, const uint64_t (&raw)[WAYS][kUnroll]) {
      const _Float16 *xa = reinterpret_cast<const _Float16 *>(sm.xs);
      const uint32_t ml = (lane & 15u) % MR;
#pragma unroll
      for (int j = 0; j < kUnroll / 4; ++j) {
        const uint32_t off = ((((kb >> 6) + j) * 16u + my_first) * MR + ml) * 4u;
        f16x4 a[3];
#pragma unroll
        for (int q = 0; q < 3; ++q)
          a[q] = *reinterpret_cast<const f16x4 *>(xa + q * XROWS * MR + off);
        f16x4 b[WAYS][4];
#pragma unroll
        for (int w = 0; w < WAYS; ++w) {
          uint32_t lo[4], hi[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int u = 4 * j + i;
            const uint32_t kk = kb + u * RPW + my_first;
            const bool ok = EXACT || (k0 + kk < kend && col_ok);
            const uint64_t r = ok ? raw[w][u] : 0ull;
            lo[i] = (uint32_t)r;
            hi[i] = (uint32_t)(r >> 32);
          }
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const uint32_t *src = c < 2 ? lo : hi;
            const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
            const uint32_t d0 = __builtin_amdgcn_perm(src[1], src[0], sel);
            const uint32_t d1 = __builtin_amdgcn_perm(src[3], src[2], sel);
            b[w][c] = __builtin_bit_cast(f16x4, (uint64_t)d0 | ((uint64_t)d1 << 32));
          }
        }
#pragma unroll
        for (int q = 0; q < 3; ++q)
#pragma unroll
          for (int w = 0; w < WAYS; ++w)
#pragma unroll
            for (int c = 0; c < 4; ++c)
              macc[w][c] = __builtin_amdgcn_mfma_f32_16x16x16f16(a[q], b[w][c], macc[w][c], 0, 0, 0);
      }
    };

    // kchunk is a multiple of G (host contract): whole groups only.  The
    // resident grid keeps HBM busy while each wave waits on its group.
    if constexpr (MF) {
      consume_mf(0, cur);
      for (uint32_t kb = G; kb < p.kchunk; kb += G) {
        issue(kb, cur);
        consume_mf(kb, cur);
      }
    } else {
      consume(0, cur);
      for (uint32_t kb = G; kb < p.kchunk; kb += G) {
        issue(kb, cur);
        consume(kb, cur);
      }
    }

    if constexpr (MF) {
      // D rows 4*(lane/16)+i below MR, unscaled by the row's power of two.
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t m = 4u * (lane >> 4) + i;
        if (m < MR) {
          const float inv = sm.xinv[m];
#pragma unroll
          for (int w = 0; w < WAYS; ++w)
#pragma unroll
            for (int c = 0; c < 4; ++c)
              sm.red[((wave * WAYS + w) * MR + m) * TW + 4 * (lane & 15u) + c] = macc[w][c][i] * inv;
        }
      }
    } else {
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
            float *dst = &sm.red[((wave * WAYS + w) * MR + m) * TW + CPL * cp];
#pragma unroll
            for (int c = 0; c < CPL; ++c)
              dst[c] = acc[w][m][c];
          }
      }
    }
    __syncthreads();

    float part[OPT];
#pragma unroll
    for (int i = 0; i < OPT; ++i) {
      const uint32_t o = tid + i * kThreads;
      float s = 0.0f;
      if (o < OUTS) {
        s = sm.red[o];
#pragma unroll
        for (int wv = 1; wv < kWaves; ++wv)
          s += sm.red[wv * OUTS + o];
      }
      part[i] = s;
    }

    if constexpr (MODE == kStandalone) {
      if (p.kchunks > 1 && !standalone_reduce(p, tile, chunk, tiles, part, sm))
        return;
      if (fu && fu->store_mode)
        store_epilogue(p, *fu, tile, part);
      else
        epilogue(p, tile, part, sm, nullptr, 0);
    } else {
      // Decode MLP: windows other than the tile's last store tagged
      // partials and finish; the last window's unit (highest workgroup
      // id of the tile) polls them, sums windows 0..kchunks-1 in order and
      // applies the epilogue.
      uint64_t *tbuf = MODE == kProducer ? mlp->tag_a : mlp->tag_b;
      if (chunk + 1 < p.kchunks) {
        uint64_t *mine = tbuf + ((uint64_t)chunk * tiles + tile) * OUTS;
#pragma unroll
        for (int i = 0; i < OPT; ++i) {
          const uint32_t o = tid + i * kThreads;
          if (o < OUTS)
            store_word(mine + o, tag_word(part[i], tag));
        }
        return;
      }
      if (p.kchunks > 1) {
        // Poll the other windows' words with all threads (NB windows per
        // round of MPOLL loads per thread), stage them in the X window's LDS,
        // then each output adds its windows in order.
        constexpr uint32_t NB = MPOLL * kThreads / OUTS;
        static_assert(NB >= 1, "a poll round holds at least one window");
        float sum[OPT];
        for (uint32_t c0 = 0; c0 + 1 < p.kchunks; c0 += NB) {
          const uint32_t nb = min(NB, p.kchunks - 1 - c0);
          float v[MPOLL];
          poll_words<MPOLL>(
              [&](int j) {
                const uint32_t e = tid + j * kThreads;
                const bool ok = e < nb * OUTS;
                const uint32_t c = c0 + (ok ? e / OUTS : 0), o = ok ? e % OUTS : 0;
                return tbuf + ((uint64_t)c * tiles + tile) * OUTS + o;
              },
              [&](int j) { return tid + j * kThreads < nb * OUTS; }, tag, v, *mlp);
          __syncthreads(); // previous round's values consumed
#pragma unroll
          for (int j = 0; j < MPOLL; ++j)
            sm.xs[tid + j * kThreads] = v[j];
          __syncthreads();
#pragma unroll
          for (int i = 0; i < OPT; ++i) {
            const uint32_t o = tid + i * kThreads;
            if (o < OUTS)
              for (uint32_t c = 0; c < nb; ++c)
                sum[i] = (c0 + c == 0) ? sm.xs[o] : sum[i] + sm.xs[c * OUTS + o];
          }
        }
#pragma unroll
        for (int i = 0; i < OPT; ++i)
          part[i] = sum[i] + part[i];
      }
      epilogue(p, tile, part, sm, MODE == kProducer ? mlp->tag_h : mlp->tag_y, tag);
      if constexpr (MODE == kConsumer) {
        // The last down tile of the last layer advances the generation past
        // every tag of the launch: every unit has read it by then (each
        // one's hand-off words, which carry the tag, are what this tile's
        // inputs waited for, directly or through earlier layers).
        if (tid == 0 && layer + 1 == mlp->layers &&
            __hip_atomic_fetch_add(mlp->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                mlp->tiles_b - 1) {
          __hip_atomic_store(mlp->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(mlp->gen, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  }

  // Matrix-core route: stage the window's X as three f16 pieces.  Row m
  // is scaled by s_m = 2^(15 - e), e = the exponent of the window's max|x|
  // in that row (max * s_m in [2^14, 2^15)); v = x * s_m splits exactly
  // into hi = f16(v), mid = f16(v - hi), lo = f16(v - hi - mid), so the
  // pieces carry v to ~33 significant bits and values down to 2^-39 of
  // the row maximum.  f16 x f16 products are exact in the f32 MFMA
  // accumulator; the unit scales its partials by 1/s_m (exact, a power of
  // two).  Layout: piece q, then window row kk = 64t + 16i + s as
  // [t][s][m][i], so a lane's A operand (4 rows 16 apart) is one 8-byte
  // read.  A thread's values all belong to row tid % MR (256 % MR == 0).
  static TA_DEVICE void stage_split(const float (&xr)[XROWS * MR / kThreads], Smem &sm) {
    constexpr int XPT = XROWS * MR / kThreads;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t m = tid % MR;
    // Row scale from the finite values only: an infinite x must not push
    // the row's finite values past the f16 range (their hi pieces would
    // turn into +-inf and the column sums into inf - inf = NaN).
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < XPT; ++j)
      mx = __builtin_isfinite(xr[j]) ? fmaxf(mx, fabsf(xr[j])) : mx;
#pragma unroll
    for (int off = MR; off < 64; off <<= 1)
      mx = fmaxf(mx, __shfl_xor(mx, off));
    if (lane < MR)
      sm.xmax[wave * MR + lane] = mx;
    __syncthreads();
    mx = sm.xmax[m];
#pragma unroll
    for (int w = 1; w < kWaves; ++w)
      mx = fmaxf(mx, sm.xmax[w * MR + m]);
    int e = 0;
    (void)frexpf(mx, &e);
    const int sx = min(126, max(-126, 15 - e));
    const float s = ldexpf(1.0f, sx);
    if (tid < MR)
      sm.xinv[tid] = ldexpf(1.0f, -sx);
    _Float16 *xa = reinterpret_cast<_Float16 *>(sm.xs);
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
      const uint32_t kk = (tid + j * kThreads) / MR;
      const uint32_t off = ((((kk >> 6) * 16u + (kk & 15u)) * MR + m) * 4u) + ((kk >> 4) & 3u);
      const float v = xr[j] * s;
      const _Float16 h = (_Float16)v;
      // An infinite x keeps hi = inf and zero residuals, so the output is
      // +-inf (or NaN against a zero weight) as with f32 FMAs.
      const float r = __builtin_isinf((float)h) ? 0.0f : v - (float)h;
      const _Float16 md = (_Float16)r;
      xa[off] = h;
      xa[XROWS * MR + off] = md;
      xa[2 * XROWS * MR + off] = (_Float16)(r - (float)md);
    }
  }

  // Normed-A preamble (src/matmul/api.rs:213-222; the reference's row
  // kernel, shaders/matmul_row_bda_kernel.glsl:212-234): each unit
  // reduces the sum of squares of its X rows over all of K (every thread
  // strides K, fixed-order tree over the workgroup), then scales the
  // staged window values: x' = (x * s_m) * w[k], s_m = 1 / sqrt(sumsq / K
  // + eps).  The whole rows are re-read per unit; they are small and
  // L2-resident.  The X window's LDS (not yet staged) is the scratch.
  static TA_DEVICE void normalize_x(const GemvArgs &p, const float *norm_w, float norm_eps,
                                    uint32_t k0,
                                    float (&xr)[XROWS * MR / kThreads], Smem &sm,
                                    const float (&pre)[kNormPre]) {
    constexpr int XPT = XROWS * MR / kThreads;
    static_assert(XS >= kThreads, "reduction scratch");
    const uint32_t tid = threadIdx.x;
    __shared__ float scale[MR];
    for (uint32_t m = 0; m < p.rows; ++m) {
      const float *row = p.x + (uint64_t)m * p.k;
      float ss = 0.0f;
      uint32_t kk = tid;
      if constexpr (MR == 1) {
        // Values loaded before the weights (zero past K: adding 0 to the
        // non-negative sum leaves it unchanged), in the loop's order.
#pragma unroll
        for (int i = 0; i < kNormPre; ++i)
          ss = fmaf(pre[i], pre[i], ss);
        kk = tid + kNormPre * kThreads;
      }
      for (; kk < p.k; kk += kThreads) {
        const float a = COH ? coherent_load(row + kk) : row[kk];
        ss = fmaf(a, a, ss);
      }
      sm.xs[tid] = ss;
      __syncthreads();
#pragma unroll
      for (uint32_t step = kThreads / 2; step > 0; step >>= 1) {
        if (tid < step)
          sm.xs[tid] += sm.xs[tid + step];
        __syncthreads();
      }
      if (tid == 0)
        scale[m] = 1.0f / sqrtf(sm.xs[0] / (float)p.k + norm_eps);
      __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
      const uint32_t i = tid + j * kThreads;
      const uint32_t kk = i / MR, m = i % MR;
      if (i < p.kchunk * MR && m < p.rows && k0 + kk < p.k)
        xr[j] = (xr[j] * scale[m]) * norm_w[k0 + kk];
    }
  }

  // Fused store epilogue (M = 1, plain alpha * acc; host-validated): RoPE
  // of the interleaved (even, odd) output pairs with the reference's fma
  // order (shaders/matmul_row_bda_kernel.glsl:163-176), then a store to Y
  // or a scatter into the destination cache (:150-161).  Output o of the
  // tile is thread o, so its pair partner o ^ 1 is the adjacent lane.
  static TA_DEVICE void store_epilogue(const GemvArgs &p, const GemvFusion &f, uint32_t tile,
                                       const float (&part)[OPT]) {
    const uint32_t tid = threadIdx.x;
    const uint32_t pos = f.pos_base + (f.pos_addr ? *f.pos_addr : 0u);
#pragma unroll
    for (int i = 0; i < OPT; ++i) {
      const uint32_t o = tid + i * kThreads;
      const uint32_t m = o / TW, c = tile * TW + o % TW;
      const bool ok = o < OUTS && m < p.rows && c < p.n;
      float v = p.alpha * part[i];
      const float partner = __shfl_xor(v, 1);
      if (!ok)
        continue;
      if (f.store_mode != 2) {
        const uint32_t dim = c % f.head_dim;
        const uint64_t angle = ((uint64_t)pos * (f.head_dim / 2) + dim / 2) * 2;
        if (angle + 1 >= f.table_len)
          continue;
        const float cos_t = f.rope_table[angle], sin_t = f.rope_table[angle + 1];
        v = (dim & 1u) == 0 ? fmaf(v, cos_t, -partner * sin_t) : fmaf(partner, sin_t, v * cos_t);
      }
      if (f.store_mode == 1) {
        p.y[(uint64_t)m * p.n + c] = v;
      } else {
        const uint64_t idx = (uint64_t)pos * f.pos_scale +
                             (uint64_t)(c / f.head_dim) * f.stride_head +
                             (uint64_t)(c % f.head_dim) * f.stride_dim;
        if (idx >= f.dst_len)
          continue;
        if (f.store_dst_f16)
          static_cast<_Float16 *>(f.store_dst)[idx] = (_Float16)v;
        else
          static_cast<float *>(f.store_dst)[idx] = v;
      }
    }
  }

  // Standalone K-window reduction: store this window's partial; the last
  // unit of the tile to arrive (integer counter) sums windows
  // 0..kchunks-1 in order into `part` and returns true.
  static TA_DEVICE bool standalone_reduce(const GemvArgs &p, uint32_t tile, uint32_t chunk,
                                          uint32_t tiles, float (&part)[OPT], Smem &sm) {
    const uint32_t tid = threadIdx.x;
    uint32_t *counter = &p.counters[tile * TA_GEMV_COUNTER_STRIDE];
    float *mine = p.partial + ((uint64_t)chunk * tiles + tile) * OUTS;
#pragma unroll
    for (int i = 0; i < OPT; ++i) {
      const uint32_t o = tid + i * kThreads;
      if (o < OUTS)
        coherent_store(mine + o, part[i]);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      const uint32_t seen =
          __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sm.last_flag = (seen == p.kchunks - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (!sm.last_flag)
      return false;
    // Sum the windows in order 0..kchunks-1.  A batch of NB windows is
    // loaded at once (16 loads per thread, one memory round trip) into the
    // X window's LDS, which is free now; then each output adds its
    // windows sequentially.
    const uint64_t step = (uint64_t)tiles * OUTS;
    const float *tsrc = p.partial + (uint64_t)tile * OUTS;
    constexpr uint32_t NB = PSTAGE / OUTS; // windows per batch
    static_assert(NB >= 1, "staging holds at least one partial");
    float sum[OPT];
#pragma unroll
    for (int i = 0; i < OPT; ++i)
      sum[i] = 0.0f;
    for (uint32_t c0 = 0; c0 < p.kchunks; c0 += NB) {
      const uint32_t nb = min(NB, p.kchunks - c0);
      __syncthreads(); // previous batch fully consumed
      float v[PSTAGE / kThreads];
#pragma unroll
      for (int j = 0; j < PSTAGE / kThreads; ++j) {
        const uint32_t e = tid + j * kThreads;
        const bool ok = e < nb * OUTS;
        const uint32_t c = c0 + (ok ? e / OUTS : 0), o = ok ? e % OUTS : 0;
        v[j] = coherent_load(tsrc + c * step + o);
      }
#pragma unroll
      for (int j = 0; j < PSTAGE / kThreads; ++j)
        sm.xs[tid + j * kThreads] = v[j];
      __syncthreads();
#pragma unroll
      for (int i = 0; i < OPT; ++i) {
        const uint32_t o = tid + i * kThreads;
        if (o < OUTS)
          for (uint32_t c = 0; c < nb; ++c)
            sum[i] = (c0 + c == 0) ? sm.xs[o] : sum[i] + sm.xs[c * OUTS + o];
      }
    }
#pragma unroll
    for (int i = 0; i < OPT; ++i)
      part[i] = sum[i];
    if (tid == 0)
      __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
  }

  // Epilogue (shaders/matmul_epilogue_common.glsl:14-21 order) on the
  // tile's K-summed outputs.  Dual mode writes U and Y; with `h_tag` it
  // also publishes Y as tagged words [col][MR] (for the decode MLP's down
  // units, or, from a down unit, for the next chained layer).  A decode-MLP
  // down unit reads Y_old and D, which earlier chained layers may have
  // written in this launch, and writes Y, which later ones may read, with
  // agent-scope accesses.
  static TA_DEVICE void epilogue(const GemvArgs &p, uint32_t tile, const float (&part)[OPT],
                                 Smem &sm, uint64_t *h_tag, uint32_t tag) {
    const uint32_t tid = threadIdx.x;
    if constexpr (DUAL) {
      __syncthreads();
#pragma unroll
      for (int i = 0; i < OPT; ++i) {
        const uint32_t o = tid + i * kThreads;
        if (o < OUTS)
          sm.red[o] = part[i];
      }
      __syncthreads();
      for (uint32_t o = tid; o < MR * TW; o += kThreads) {
        const uint32_t m = o / TW, c = tile * TW + o % TW;
        if (m >= p.rows || c >= p.n)
          continue;
        const uint64_t yi = (uint64_t)m * p.n + c;
        const float u = p.alpha * sm.red[MR * TW + o];
        float g = p.alpha * sm.red[o];
        if (p.flags & TA_FLAG_BIAS)
          g += p.bias[c];
        const float h = ta_activate(g, p.act) * u;
        if constexpr (MODE == kStandalone) {
          p.y2[yi] = u;
          p.y[yi] = h;
        } else {
          // Agent-scope stores: a later chained layer may rewrite or read
          // these buffers.
          coherent_store(p.y2 + yi, u);
          coherent_store(p.y + yi, h);
        }
        if (h_tag)
          store_word(h_tag + (uint64_t)c * MR + m, tag_word(h, tag));
      }
    } else {
#pragma unroll
      for (int i = 0; i < OPT; ++i) {
        const uint32_t o = tid + i * kThreads;
        const uint32_t m = o / TW, c = tile * TW + o % TW;
        if (o >= OUTS || m >= p.rows || c >= p.n)
          continue;
        const uint64_t yi = (uint64_t)m * p.n + c;
        constexpr bool kCoherent = MODE == kConsumer || COH;
        auto rd = [&](const float *q) { return kCoherent ? coherent_load(q) : *q; };
        float v = p.alpha * part[i];
        if (p.flags & TA_FLAG_ACCUMULATE)
          v += rd(p.y + yi);
        if (p.flags & TA_FLAG_BIAS)
          v += p.bias[c];
        v = ta_activate(v, p.act);
        if (p.binary == TA_BIN_ADD_SCALED)
          v = fmaf(p.beta, rd(p.d + yi), v);
        else if (p.binary == TA_BIN_MUL)
          v *= rd(p.d + yi);
        if constexpr (kCoherent) {
          coherent_store(p.y + yi, v);
          if (h_tag)
            store_word(h_tag + (uint64_t)c * MR + m, tag_word(v, tag));
        } else {
          p.y[yi] = v;
        }
      }
    }
  }

  static TA_DEVICE void run(const GemvArgs &p, const GemvFusion &f) {
    __shared__ __attribute__((aligned(16))) Smem sm;
    const uint32_t tiles = (p.n + TW - 1) / TW;
    unit(p, blockIdx.x % tiles, blockIdx.x / tiles, sm, nullptr, 0, &f);
  }
};

// Rows of X staged per standalone unit: 16 KiB of LDS.
template <int MR> constexpr int standalone_rows() { return 4096 / MR; }
// Standalone launches with 4 or 8 rows load groups of 8 per matrix (their
// accumulators take the registers a deeper group would: 8 rows of a dual
// launch then fit 3 workgroups per CU instead of 2); 1 and 2 rows load
// groups of 16.  The host's gemv_unit() mirrors this group size.
template <int MR> constexpr int standalone_unroll() { return MR >= 4 ? 8 : 16; }

// Persistent decode MLP chain.  Per layer, the first units_a workgroups run
// gate/up (producer) units, the rest down-proj (consumer) units; layers
// follow each other in workgroup id.  Every wait is on units with lower
// workgroup ids (down units on gate/up units of their layer; gate/up units
// on the previous layer's down units; the last K window of a tile, which has
// the tile's highest id, on the tile's other windows), and workgroups are
// dispatched in id order, so a waited-on unit has always been dispatched and
// never waits on its waiter; the bounded wait is a safety net only.  A
// layer's gate/up units are dispatched as the previous layer's gate/up units
// exit and issue their weight reads before waiting for their x, so HBM
// streams the next layer's weights through the previous layer's hand-off
// tail.  No launch-wide counter is touched at
// unit start (one hot atomic would serialise the starts).
// K windows: gate/up units take 256 rows (one group of 16 loads per
// matrix), down units 256 rows too (one group of 16 loads; 512-row down
// windows, half as many units, measured the same at one row and 1-2%
// slower at four and eight).
constexpr int kMlpRowsA = TA_MLP_ROWS_A;
constexpr int kMlpRowsB = TA_MLP_ROWS_B;
static_assert(kMlpRowsA % 256 == 0 && kMlpRowsB % 256 == 0, "whole groups of 16 loads");

template <int MR> struct DecodeMlp {
  typedef Gemv<MR, true, 64, false, kProducer, kMlpRowsA, kMlpRowsA / 16> A;
  typedef Gemv<MR, false, 64, false, kConsumer, kMlpRowsB, kMlpRowsB / 16> B;
  union Smem {
    typename A::Smem a;
    typename B::Smem b;
  };

  static TA_DEVICE void run(const MlpArgs &p) {
    __shared__ __attribute__((aligned(16))) Smem sm;
    const uint32_t per_layer = p.units_a + p.units_b;
    const uint32_t layer = blockIdx.x / per_layer, r = blockIdx.x % per_layer;
    if (r < p.units_a)
      A::unit(p.layer[layer].a, r % p.tiles_a, r / p.tiles_a, sm.a, &p, layer);
    else
      B::unit(p.layer[layer].b, (r - p.units_a) % p.tiles_b, (r - p.units_a) / p.tiles_b, sm.b, &p,
              layer);
  }
};

} // namespace

namespace {
// The row-major f16 decode GEMV at one row (ta_gemv_f16_t64_m1's unit).
using ChainGemv =
    Gemv<1, false, 64, false, kStandalone, standalone_rows<1>(), standalone_unroll<1>(), true>;

// Grid barrier of the chain: every thread waits for its agent-scope
// (write-through) output stores to complete, thread 0 reads the
// generation, waits for that value, counts the workgroup in; the last to
// arrive resets the count and advances the generation, the others poll it.
// Readers use agent-scope loads, so no cache-wide fence is needed (an
// agent-scope fence writes back and invalidates the whole L2 of the XCD,
// which measured ~40 us per barrier here).  Every workgroup of the launch arrives (a workgroup not yet
// resident waits only for CUs held by kernels that finish on their own),
// so the bound is a safety net: past it the wait raises the host-visible
// status word and the workgroup stops.
TA_DEVICE bool chain_barrier(const GemvChainArgs &c, uint32_t &flag) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t *count = c.barrier, *gen = c.barrier + TA_GEMV_COUNTER_STRIDE;
    uint32_t g0 = __hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(g0) : : "memory");
    uint32_t ok = 1;
    if (__hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
        gridDim.x - 1) {
      __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(gen, g0 + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      for (uint32_t polls = 0;
           __hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == g0;) {
        if (++polls >= c.spin_limit) {
          __hip_atomic_store(c.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
          ok = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    flag = ok;
  }
  __syncthreads();
  return flag != 0;
}
} // namespace

extern "C" __global__ __launch_bounds__(kThreads) void
ta_gemv_chain_f16_m1(GemvChainArgs c) {
  __shared__ __attribute__((aligned(16))) ChainGemv::Smem sm;
  __shared__ uint32_t flag;
  for (uint32_t j0 = 0; j0 < c.n_jobs;) {
    uint32_t j1 = j0;
    while (j1 + 1 < c.n_jobs && !((c.sync_after >> j1) & 1u))
      ++j1;
    // Units of the group's jobs, laid end to end (constant indices into
    // the argument arrays: no private copy of them).
    uint32_t first[TA_GEMV_CHAIN_MAX_JOBS], total = 0;
#pragma unroll
    for (int q = 0; q < TA_GEMV_CHAIN_MAX_JOBS; ++q) {
      first[q] = total;
      if ((uint32_t)q >= j0 && (uint32_t)q <= j1)
        total += c.units[q];
    }
    for (uint32_t u = blockIdx.x; u < total; u += gridDim.x) {
      uint32_t j = j0;
#pragma unroll
      for (int q = 1; q < TA_GEMV_CHAIN_MAX_JOBS; ++q)
        if ((uint32_t)q > j0 && (uint32_t)q <= j1 && u >= first[q])
          j = q;
      uint32_t lu = u;
#pragma unroll
      for (int q = 0; q < TA_GEMV_CHAIN_MAX_JOBS; ++q)
        if ((uint32_t)q == j)
          lu = u - first[q];
      const GemvArgs &p = c.job[j];
      const uint32_t tiles = (p.n + 63) / 64;
      ChainGemv::unit(p, lu % tiles, lu / tiles, sm, nullptr, 0, &c.fu[j]);
      __syncthreads(); // the next unit reuses the LDS
    }
    if (j1 + 1 >= c.n_jobs)
      break;
    if (!chain_barrier(c, flag))
      return;
    j0 = j1 + 1;
  }
}

#define TA_GEMV(NAME, MR, DUAL, TW, WF32)                                          \
  extern "C" __global__ __launch_bounds__(kThreads) void NAME(GemvArgs p,          \
                                                              GemvFusion f) {      \
    Gemv<MR, DUAL, TW, WF32, kStandalone, standalone_rows<MR>(),                  \
         standalone_unroll<MR>()>::run(p, f);                                     \
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

// WAVES: waves per SIMD the register budget must allow, so every
// workgroup of the launch can be resident (4: <= 128 VGPRs, 3: <= 168).
#define TA_MLP(MR, WAVES)                                                          \
  extern "C" __global__ __launch_bounds__(kThreads)                                \
      __attribute__((amdgpu_waves_per_eu(WAVES))) void ta_decode_mlp_f16_t64_m##MR( \
          MlpArgs p) {                                                             \
    DecodeMlp<MR>::run(p);                                                         \
  }
TA_MLP(1, 4)
TA_MLP(2, 4)
TA_MLP(4, 4)
TA_MLP(8, 3)
