// f16-MFMA GEMM with f32 accumulation, for gfx950 (CDNA4).
//
// Replaces the reference's tensor-core GEMMs
// (shaders/matmul_coopmat_kernel.glsl:1-27 f16w / a16 coopmat and
// matmul_cm2_kernel.glsl:1-49 with its fused epilogue).  Same numerics:
// B is f16 storage; A is f32 rounded to f16 (RNE) when it is staged, or
// f16 storage (the a16 route); products are exact in the f32 accumulator;
// C is f32 with the full fused epilogue, or f16 (RNE) for the a16 route.
//
// Design (one workgroup per BM x BN tile, 4 waves in a 2x2 grid):
//  * v_mfma_f32_32x32x16_f16: a wave owns FM x FN blocks of 32x32.  Each
//    lane feeds 8 consecutive k of its A row and the same 8 k of its B
//    column per instruction, so both operands are staged k-contiguous in
//    LDS: As[m][k] and Bs[n][k] (+8 halves pad), one 128-bit read each.
//  * B arrives [K][N] (n contiguous) and is transposed while staging: a
//    thread loads a 4x4 block (four 64-bit row pieces) and writes four
//    64-bit k-runs.  A (f32) is converted with v_cvt_f16_f32 (RNE).
//  * K slabs of 64 (four MFMA k-steps), two LDS buffers + one register
//    stage, one barrier per slab (as in gemm_f32.hip); the shared output
//    stage applies the epilogue with coalesced stores.
#include "common.h"

namespace {

template <int BM, int BN, int WGM, int WGN, bool VEC, bool A_F16>
struct GemmH16 {
  static constexpr int BK = 64;
  static constexpr int T = 64 * WGM * WGN;
  static constexpr int WTM = BM / WGM, WTN = BN / WGN;
  static constexpr int FM = WTM / 32, FN = WTN / 32;
  static constexpr int LDK = BK + 8; // halves per staged row (+16 B pad)
  static constexpr int A_STAGE = BM * LDK, B_STAGE = BN * LDK; // halves
  static constexpr int STAGE = A_STAGE + B_STAGE;
  // A slab: BM x BK in 4-wide k pieces; B slab: (BK/4) x (BN/4) 4x4 blocks.
  static constexpr int A_PER = BM * BK / 4 / T;
  static constexpr int B_PER = (BK / 4) * (BN / 4) / T;
  static_assert(A_PER * T * 4 == BM * BK, "A slab splits evenly");
  static_assert(B_PER * T == (BK / 4) * (BN / 4), "B slab splits evenly");
  static_assert(FM >= 1 && FN >= 1, "wave tile must be a multiple of 32");
  static constexpr int SMEM_FLOATS = (2 * STAGE + 1) / 2;
  static_assert(T / 64 * 32 * (WTN + 4) <= SMEM_FLOATS, "C staging fits in LDS");

  typedef typename std::conditional<A_F16, const _Float16, const float>::type AT;

  static TA_DEVICE void load_a(AT *A, uint32_t M, uint32_t K, uint32_t m0, uint32_t k0,
                               bool full, uint32_t tid, f16x4 (&ra)[A_PER]) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const uint32_t e = tid + i * T;
      const uint32_t row = e / (BK / 4), kq = e % (BK / 4);
      const uint32_t gm = m0 + row, gk = k0 + kq * 4;
      AT *src = A + (uint64_t)gm * K + gk;
      if (VEC && full) {
        if constexpr (A_F16) {
          ra[i] = *reinterpret_cast<const f16x4 *>(src);
        } else {
          const f32x4 v = *reinterpret_cast<const f32x4 *>(src);
          ra[i] = f16x4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
        }
      } else {
        f16x4 v = {0, 0, 0, 0};
        if (gm < M) {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (gk + c < K)
              v[c] = (_Float16)src[c];
        }
        ra[i] = v;
      }
    }
  }

  // 4x4 block (k4, n4): rows k0+4*k4+r, columns n0+4*n4+c.
  static TA_DEVICE void load_b(const _Float16 *B, uint32_t N, uint32_t K, uint32_t n0, uint32_t k0,
                               bool full, uint32_t tid, f16x4 (&rb)[B_PER][4]) {
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const uint32_t e = tid + i * T;
      const uint32_t n4 = e % (BN / 4), k4 = e / (BN / 4);
      const uint32_t gn = n0 + n4 * 4;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t gk = k0 + k4 * 4 + r;
        const _Float16 *src = B + (uint64_t)gk * N + gn;
        if (VEC && full) {
          rb[i][r] = *reinterpret_cast<const f16x4 *>(src);
        } else {
          f16x4 v = {0, 0, 0, 0};
          if (gk < K) {
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (gn + c < N)
                v[c] = src[c];
          }
          rb[i][r] = v;
        }
      }
    }
  }

  static TA_DEVICE void store_lds(_Float16 *As, _Float16 *Bs, uint32_t tid, const f16x4 (&ra)[A_PER],
                                  const f16x4 (&rb)[B_PER][4]) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const uint32_t e = tid + i * T;
      *reinterpret_cast<f16x4 *>(&As[(e / (BK / 4)) * LDK + (e % (BK / 4)) * 4]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const uint32_t e = tid + i * T;
      const uint32_t n4 = e % (BN / 4), k4 = e / (BN / 4);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f16x4 col = {rb[i][0][c], rb[i][1][c], rb[i][2][c], rb[i][3][c]};
        *reinterpret_cast<f16x4 *>(&Bs[(n4 * 4 + c) * LDK + k4 * 4]) = col;
      }
    }
  }

  static TA_DEVICE void compute(const _Float16 *As, const _Float16 *Bs, uint32_t lane, uint32_t wm,
                                uint32_t wn, f32x16 (&acc)[FM][FN]) {
    const uint32_t lr = lane & 31u, lg = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      f16x8 a[FM], b[FN];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        a[fm] = *reinterpret_cast<const f16x8 *>(&As[(wm * WTM + fm * 32 + lr) * LDK + ks * 16 + lg * 8]);
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
        b[fn] = *reinterpret_cast<const f16x8 *>(&Bs[(wn * WTN + fn * 32 + lr) * LDK + ks * 16 + lg * 8]);
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
          acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[fm], b[fn], acc[fm][fn], 0, 0, 0);
    }
  }

  static TA_DEVICE void run(const GemmArgs &p) {
    __shared__ __attribute__((aligned(16))) float smem[SMEM_FLOATS];
    _Float16 *sh = reinterpret_cast<_Float16 *>(smem);
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t wm = wave / WGN, wn = wave % WGN;
    uint32_t tm, tn;
    ta_tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t batch = blockIdx.z;
    AT *A = static_cast<AT *>(p.a) + (uint64_t)batch * p.stride_a;
    const _Float16 *B = static_cast<const _Float16 *>(p.b) + (uint64_t)batch * p.stride_b;
    const bool mn_full = (m0 + BM <= p.m) && (n0 + BN <= p.n);

    f32x16 acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          acc[fm][fn][r] = 0.0f;

    const uint32_t kts = (p.k + BK - 1) / BK;
    f16x4 ra[A_PER], rb[B_PER][4];
    {
      const bool full = mn_full && BK <= p.k;
      load_a(A, p.m, p.k, m0, 0, full, tid, ra);
      load_b(B, p.n, p.k, n0, 0, full, tid, rb);
      store_lds(sh, sh + A_STAGE, tid, ra, rb);
    }
    __syncthreads();
    for (uint32_t kt = 0; kt < kts; ++kt) {
      _Float16 *cur = sh + (kt & 1u) * STAGE;
      const bool more = kt + 1 < kts;
      if (more) {
        const uint32_t k0 = (kt + 1) * BK;
        const bool full = mn_full && k0 + BK <= p.k;
        load_a(A, p.m, p.k, m0, k0, full, tid, ra);
        load_b(B, p.n, p.k, n0, k0, full, tid, rb);
      }
      compute(cur, cur + A_STAGE, lane, wm, wn, acc);
      if (more) {
        _Float16 *nx = sh + ((kt + 1) & 1u) * STAGE;
        store_lds(nx, nx + A_STAGE, tid, ra, rb);
      }
      __syncthreads();
    }
    ta_store_tile<WTM, WTN, FM, FN, T, A_F16>(smem, SMEM_FLOATS, acc, p, lane, wave, wm, wn, m0, n0,
                                              batch, 0);
  }
};


// ---------------------------------------------------------------------
// Pipelined f16 x f16 GEMM (both operands f16 in memory), the fast path
// for K % 64 == 0 and N % 8 == 0.  The f16w route gets its f16 A from
// ta_cvt_f32_f16 (RNE, the same rounding as staging-time conversion), the
// a16 route reads its A directly.  Serves the plain tiles
// (ta_gemm_{h16,a16}_<tile>_lds, k_splits = 1) and the split-K tiles
// (ta_gemm_h16sk_<tile>).
//
//  * Two pipeline levels (DBUF; the 256 x 256 tile has room for two LDS
//    stages only and runs the one-level loop).  Global -> LDS: gfx950's direct loads
//    (global_load_lds_dwordx4, no register staging), NS stages of 64 k,
//    one barrier per stage.  LDS -> registers: the MFMA fragments of stage
//    kt + 1 are read into a second register set while the MFMAs of stage
//    kt run, so a stage costs about max(MFMA chain, LDS reads + barrier)
//    rather than their sum.  At iteration kt a wave waits until stage
//    kt + 1 has landed (NS - 3 newer stages may still be in flight), joins
//    the barrier, refills the buffer of stage kt - 1 (its fragments were
//    consumed in iteration kt - 1) with stage kt + NS - 1, reads stage kt +
//    1's fragments and runs stage kt's MFMAs.  The loads are issued from
//    inline asm with explicit vmcnt waits: the compiler would otherwise
//    wait for every outstanding direct load before each LDS read.
//  * A stage: As[m][64] f16, B stage: Bs[64][BN] f16 exactly as B lies in
//    memory (n contiguous).  A wave instruction writes 1 KiB of LDS
//    contiguously (lane l at +16 l), so the bank-conflict swizzles are
//    applied to which 16-byte global chunk a lane fetches: LDS slot c of
//    row r holds global chunk c ^ swz(r).
//  * Waves: WGM x WGN, each owning a WTM x WTN sub-tile of FM x FN MFMA
//    blocks of 32x32 (v_mfma_f32_32x32x16_f16).  8 waves (two per SIMD)
//    for tiles of 128 x 64 and larger.
//  * A operand: one ds_read_b128 per 32x32x16 MFMA (row, 8 k).  B operand:
//    two ds_read_b64_tr_b16 (the CDNA4 LDS transpose read): in each group
//    of 16 lanes, lane i receives element i % 4 of the 8-byte pieces the
//    group's lanes 4j + i / 4 address (j = 0..3), so addressing row
//    k0 + t / 4, columns nb + 4 (t % 4) from lane t hands lane i the
//    column nb + i over rows k0..k0+3 - the MFMA's B layout, read from a
//    row-major tile.
//  * Rows past M and column chunks past N read clamped (valid) addresses:
//    their products only reach outputs the store guards drop.
//  * Split-K (k_splits = S > 1, blockIdx.y = split s): split s takes K
//    stages [lo, hi), lo = s * (steps / S) + min(s, steps % S) (the split
//    window rule of the reference's split-K, in whole stages).  Every split
//    stores its raw f32 accumulators to its slot of `partial` (lane-major,
//    8-byte agent-scope stores, visible across the XCD L2s), waits for
//    them, and increments the tile's counter.  The workgroup that brings
//    the count to S sums the S partials in split order 0..S-1 (its own
//    from registers, the others with agent-scope loads), so the result does
//    not depend on which split finished last; then it runs the fused
//    epilogue and clears the counter.  Nothing waits on another workgroup,
//    so any residency order completes.  Used for deep K, where a tile's
//    chain of stages is long and the grid small.
template <int BM, int BN, int BK, int WGM, int WGN, int NS, bool C_F16, bool SPLIT, bool DBUF,
          bool DUAL = false>
struct GemmH16Pipe {
  static constexpr int T = 64 * WGM * WGN;
  static constexpr int WAYS = DUAL ? 2 : 1; // weight matrices streamed per stage
  static constexpr int WTM = BM / WGM, WTN = BN / WGN;
  static constexpr int FM = WTM / 32, FN = WTN / 32;
  static constexpr int KS = BK / 16; // MFMA k-steps per stage
  static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BK * BN * 2;
  static constexpr int STAGE = A_BYTES + WAYS * B_BYTES;
  static constexpr int CPA = BK / 8, CPR = BN / 8; // 16-byte chunks per A / B row
  static constexpr int A_LD = A_BYTES / 16 / T, B_LD = B_BYTES / 16 / T;
  static constexpr int LD = A_LD + WAYS * B_LD; // direct loads per thread per stage
  static_assert(!DUAL || (!SPLIT && !C_F16), "dual: f32 C, no split-K");
  static_assert(A_LD * T * 16 == A_BYTES && B_LD * T * 16 == B_BYTES, "stages split evenly");
  static_assert(CPR >= 8, "B swizzle needs >= 8 chunks per row");
  static_assert(BK == 32 || BK == 64, "A rows of 4 or 8 chunks");
  static_assert(FM >= 1 && FN >= 1, "wave tile must be a multiple of 32");
  static constexpr int SMEM_BYTES = NS * STAGE;
  static_assert(SMEM_BYTES <= 160 * 1024 - 256, "LDS");
  static_assert(WGM * WGN * 32 * (WTN + 4) * 4 <= SMEM_BYTES, "C staging fits in LDS");
  static_assert(NS >= (DBUF ? 3 : 2) && (NS - 2) * LD <= 63, "vmcnt range");

  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  typedef __attribute__((address_space(3))) f16x8 lds_f16x8;

  // Swizzles (in 16-byte chunks), conflict-free whether the LDS serves
  // 128 or 256 bytes per cycle.  A (ds_read_b128, 8 or 16 lanes per
  // cycle on consecutive rows, one chunk column): the rows' chunks must
  // land in distinct slots modulo 8 for 8 consecutive rows and in distinct
  // (row parity, slot) pairs for 16.  B (transpose reads, 16 or 32 lanes
  // per cycle on 4 consecutive rows x 2 or 4 chunks): row j of the four
  // is XORed with a pattern that separates the rows in chunk bits (b1,b2)
  // and in (b2,b3) - for 8-chunk rows, bit b2 together with the row parity.
  // BK = 32 (4-chunk A rows, 4 rows per 256-byte bank line): the slot is
  // c ^ (((row >> 1) ^ (row >> 2)) & 3).  Chosen by measurement: the
  // pattern c ^ (((row >> 1) ^ (row >> 3)) & 3), which separates 8 and 16
  // consecutive rows just as well on paper, stalled the dual 128 x 128
  // tile's LDS on bank conflicts for a third of its active cycles
  // (SQ_LDS_BANK_CONFLICT 1.5 M against 0.09 M cycles), as did
  // (row >> 1) & 3; (row ^ (row >> 2)) & 3 and (row >> 2) & 3 measured
  // conflict-free too.
  static TA_DEVICE uint32_t swz_a(uint32_t row) {
    return CPA == 8 ? (row & 7u) ^ ((row >> 3) & 1u) : ((row >> 1) ^ (row >> 2)) & 3u;
  }
  static TA_DEVICE uint32_t swz_b(uint32_t row) {
    return CPR >= 16 ? (0xACA60u >> (4u * (row & 3u))) & 15u : 2u * (row & 3u);
  }

  static TA_DEVICE void load16(const void *src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
                 : "memory", "m0");
  }

  struct Frags {
    f16x8 a[KS][FM], b[WAYS][KS][FN];
  };

  static TA_DEVICE void read_frags(uint32_t st, const uint32_t (&a_off)[KS][FM],
                                   const uint32_t (&b_off)[KS][FN][2], Frags &f) {
#pragma unroll
    for (int j = 0; j < KS; ++j) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        f.a[j][fm] = *(lds_f16x8 *)(uintptr_t)(st + a_off[j][fm]);
#pragma unroll
      for (int w = 0; w < WAYS; ++w)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4 *)(uintptr_t)(st + w * B_BYTES + b_off[j][fn][0]));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4 *)(uintptr_t)(st + w * B_BYTES + b_off[j][fn][1]));
          f.b[w][j][fn] =
              __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
    }
  }

  // acc2: the second weight matrix's accumulators (dual launches only).
  static TA_DEVICE void mfmas(const Frags &f, f32x16 (&acc)[FM][FN],
                              f32x16 (&acc2)[DUAL ? FM : 1][DUAL ? FN : 1]) {
#pragma unroll
    for (int j = 0; j < KS; ++j)
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[j][fm], f.b[0][j][fn],
                                                               acc[fm][fn], 0, 0, 0);
          if constexpr (DUAL)
            acc2[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[j][fm], f.b[1][j][fn],
                                                                  acc2[fm][fn], 0, 0, 0);
        }
  }

  static TA_DEVICE void run(const GemmArgs &p) {
    __shared__ __attribute__((aligned(1024))) char smem[SMEM_BYTES];
    __shared__ uint32_t last_flag;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave / WGN, wn = wave % WGN;
    uint32_t tm, tn;
    ta_tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t batch = blockIdx.z, split = blockIdx.y;
    const uint32_t S = SPLIT && p.k_splits > 1 ? p.k_splits : 1u;
    const _Float16 *A = static_cast<const _Float16 *>(p.a) + (uint64_t)batch * p.stride_a;
    const _Float16 *B = static_cast<const _Float16 *>(p.b) + (uint64_t)batch * p.stride_b;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)smem;

    const uint32_t steps = p.k / BK, per = steps / S, extra = steps % S;
    const uint32_t klo = split * per + min(split, extra);
    const uint32_t kts = per + (split < extra ? 1u : 0u);

    // Per-thread source pointers of its direct loads (advanced per stage).
    const char *asrc[A_LD];
    const char *bsrc[WAYS][B_LD];
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const uint32_t q = i * T + tid, row = q / CPA, c = (q % CPA) ^ swz_a(row);
      const uint32_t gm = min(m0 + row, p.m - 1);
      asrc[i] = reinterpret_cast<const char *>(A + (uint64_t)gm * p.k + (uint64_t)klo * BK + 8 * c);
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const uint32_t q = i * T + tid, row = q / CPR, c = (q % CPR) ^ swz_b(row);
      const uint32_t gn = min(n0 + 8 * c, p.n - 8);
      const uint64_t off = ((uint64_t)klo * BK + row) * p.n + gn;
      bsrc[0][i] = reinterpret_cast<const char *>(B + off);
      if constexpr (DUAL)
        bsrc[1][i] = reinterpret_cast<const char *>(
            static_cast<const _Float16 *>(p.b2) + (uint64_t)batch * p.stride_b + off);
    }
    const uint64_t b_step = (uint64_t)BK * p.n * 2;

    auto issue = [&](uint32_t stage) {
      const uint32_t base = lds0 + stage * STAGE + wave * 64 * 16;
#pragma unroll
      for (int i = 0; i < A_LD; ++i) {
        load16(asrc[i], base + i * T * 16);
        asrc[i] += BK * 2;
      }
#pragma unroll
      for (int w = 0; w < WAYS; ++w)
#pragma unroll
        for (int i = 0; i < B_LD; ++i) {
          load16(bsrc[w][i], base + A_BYTES + w * B_BYTES + i * T * 16);
          bsrc[w][i] += b_step;
        }
    };

    // Per-lane LDS read offsets within a stage.
    const uint32_t lr = lane & 31u, lg = lane >> 5;
    uint32_t a_off[KS][FM];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const uint32_t row = wm * WTM + fm * 32 + lr;
        a_off[ks][fm] = row * (BK * 2) + 16u * ((2u * ks + lg) ^ swz_a(row));
      }
    const uint32_t g = lane >> 4, t = lane & 15u;
    uint32_t b_off[KS][FN][2];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          const uint32_t row = ks * 16 + 8 * (g >> 1) + 4 * rr + (t >> 2);
          const uint32_t col = wn * WTN + fn * 32 + 16 * (g & 1u) + 4 * (t & 3u);
          b_off[ks][fn][rr] = A_BYTES + row * (BN * 2) + 16u * ((col >> 3) ^ swz_b(row)) +
                             (col & 7u) * 2;
        }

    f32x16 acc[FM][FN];
    f32x16 acc2[DUAL ? FM : 1][DUAL ? FN : 1];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          acc[fm][fn][r] = 0.0f;
          if constexpr (DUAL)
            acc2[fm][fn][r] = 0.0f;
        }

#pragma unroll
    for (int s = 0; s < NS - 1; ++s)
      if (s < (int)kts)
        issue(s);

    if constexpr (!DBUF) {
      // One register set: wait for stage kt, barrier, refill, read, MFMAs
      // (the 256 x 256 tile: two 64 KiB stages leave no room for a third;
      // the dual 128 x 128 tile at 16 waves, whose second set would spill).
      for (uint32_t kt = 0; kt < kts; ++kt) {
        if (kt + NS - 2 < kts)
          asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NS - 2) * LD) : "memory");
        else
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (kt + NS - 1 < kts)
          issue((kt + NS - 1) % NS);
        Frags f;
        read_frags(lds0 + (kt % NS) * STAGE, a_off, b_off, f);
        mfmas(f, acc, acc2);
      }
    } else {
    Frags fr[2];
    if (kts > 0) {
      // stage 0 landed: min(NS - 2, kts - 1) newer stages may be in flight
      if (kts >= NS - 1)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NS - 2) * LD) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      read_frags(lds0, a_off, b_off, fr[0]);
    }
    // Two iterations per trip so the register sets are fixed (no dynamic
    // indexing of fr).
    auto step = [&](uint32_t kt, Frags &cur, Frags &nxt) __attribute__((always_inline)) {
      if (kt + 1 < kts) {
        if (kt + NS - 2 < kts)
          asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NS - 3) * LD) : "memory");
        else
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      __syncthreads();
      if (kt + NS - 1 < kts)
        issue((kt + NS - 1) % NS);
      if (kt + 1 < kts)
        read_frags(lds0 + ((kt + 1) % NS) * STAGE, a_off, b_off, nxt);
      mfmas(cur, acc, acc2);
    };
    uint32_t kt = 0;
    for (; kt + 1 < kts; kt += 2) {
      step(kt, fr[0], fr[1]);
      step(kt + 1, fr[1], fr[0]);
    }
    if (kt < kts)
      step(kt, fr[0], fr[1]);
    }
    __syncthreads();

    if (SPLIT && S > 1) {
      const uint64_t tile_id = (uint64_t)batch * p.tiles_m * p.tiles_n + blockIdx.x;
      uint64_t *slots = reinterpret_cast<uint64_t *>(p.partial) + tile_id * S * (BM * BN / 2);
      uint64_t *mine = slots + (uint64_t)split * (BM * BN / 2);
#pragma unroll
      for (int f = 0; f < FM * FN; ++f)
#pragma unroll
        for (int r2 = 0; r2 < 8; ++r2) {
          // Element values are copied out first: a bit cast of a vector
          // element lvalue reads the vector's first element in this clang.
          const float lo = acc[f / FN][f % FN][2 * r2], hi = acc[f / FN][f % FN][2 * r2 + 1];
          const uint64_t w = (uint64_t)__float_as_uint(lo) | ((uint64_t)__float_as_uint(hi) << 32);
          __hip_atomic_store(mine + (uint64_t)(f * 8 + r2) * T + tid, w, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
      // Publication.  Partials, counter and the last arriver's reads are
      // all agent-scope atomics (sc1: performed at the device-coherent
      // level, never from a stale L2 line).  Every thread's partial stores
      // have completed (vmcnt(0)) before the barrier, the counter increment
      // is issued after it, and the reads are issued only once the
      // increment's returned value, broadcast through the second barrier,
      // has named this workgroup the last; the barriers' workgroup fences
      // keep the compiler from moving the atomics across them.  An
      // agent-scope release on the increment plus an acquire fence in the
      // last arriver (an L2 write-back and invalidate) measured 35.3 ->
      // 39.8 us on the 512x2048x5632 down projection, so the ordering rests
      // on the completed stores instead.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      uint32_t *counter = p.counters + tile_id * TA_GEMV_COUNTER_STRIDE;
      if (tid == 0)
        last_flag =
            __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
      __syncthreads();
      if (!last_flag)
        return;
      // Fixed split order: acc = ((p0 + p1) + p2) + ...
      f32x16 tot[FM][FN];
      for (uint32_t j = 0; j < S; ++j) {
        f32x16 src[FM][FN];
        if (j == split) {
#pragma unroll
          for (int f = 0; f < FM * FN; ++f)
            src[f / FN][f % FN] = acc[f / FN][f % FN];
        } else {
          const uint64_t *from = slots + (uint64_t)j * (BM * BN / 2);
#pragma unroll
          for (int f = 0; f < FM * FN; ++f)
#pragma unroll
            for (int r2 = 0; r2 < 8; ++r2) {
              const uint64_t w =
                  __hip_atomic_load(const_cast<uint64_t *>(from) + (uint64_t)(f * 8 + r2) * T + tid,
                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              src[f / FN][f % FN][2 * r2] = __uint_as_float((uint32_t)w);
              src[f / FN][f % FN][2 * r2 + 1] = __uint_as_float((uint32_t)(w >> 32));
            }
        }
#pragma unroll
        for (int f = 0; f < FM * FN; ++f)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            tot[f / FN][f % FN][r] = j == 0 ? src[f / FN][f % FN][r]
                                            : tot[f / FN][f % FN][r] + src[f / FN][f % FN][r];
      }
#pragma unroll
      for (int f = 0; f < FM * FN; ++f)
        acc[f / FN][f % FN] = tot[f / FN][f % FN];
      if (tid == 0)
        __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if constexpr (DUAL) {
      // U = alpha * (A @ B2) first, to c2 with no epilogue; then the
      // gate's fused epilogue, whose D = c2 reads U back.  Both stores map
      // element (row, col) to the same thread, so each U value is read
      // back by the thread that stored it.
      GemmArgs pu = p;
      pu.c = p.c2;
      pu.c16 = nullptr;
      pu.flags = 0;
      pu.act = TA_ACT_NONE;
      pu.binary = TA_BIN_NONE;
      ta_store_tile<WTM, WTN, FM, FN, T, false>(reinterpret_cast<float *>(smem), SMEM_BYTES / 4,
                                                acc2, pu, lane, wave, wm, wn, m0, n0, batch, 0);
    }
    ta_store_tile<WTM, WTN, FM, FN, T, C_F16>(reinterpret_cast<float *>(smem), SMEM_BYTES / 4, acc,
                                              p, lane, wave, wm, wn, m0, n0, batch, 0);
  }
};

} // namespace

#define TA_GEMM_H16(NAME, BM, BN, WGM, WGN, VEC, A_F16)                             \
  extern "C" __global__ __launch_bounds__(64 * WGM * WGN) void NAME(GemmArgs p) {  \
    GemmH16<BM, BN, WGM, WGN, VEC, A_F16>::run(p);                                 \
  }

#define TA_GEMM_H16_FAMILY(TAG, BM, BN, WGM, WGN)                                   \
  TA_GEMM_H16(ta_gemm_h16_##TAG##_vec, BM, BN, WGM, WGN, true, false)               \
  TA_GEMM_H16(ta_gemm_h16_##TAG##_gen, BM, BN, WGM, WGN, false, false)              \
  TA_GEMM_H16(ta_gemm_a16_##TAG##_vec, BM, BN, WGM, WGN, true, true)                \
  TA_GEMM_H16(ta_gemm_a16_##TAG##_gen, BM, BN, WGM, WGN, false, true)

TA_GEMM_H16_FAMILY(m128n128, 128, 128, 2, 2)
TA_GEMM_H16_FAMILY(m128n64, 128, 64, 2, 2)
TA_GEMM_H16_FAMILY(m64n128, 64, 128, 2, 2)
TA_GEMM_H16_FAMILY(m64n64, 64, 64, 2, 2)

// Pipelined kernels: ta_gemm_h16_<tile>_lds (A pre-rounded to f16 by
// ta_cvt_f32_f16, f32 C with the fused epilogue), ta_gemm_a16_<tile>_lds
// (f16 A, f16 C) and the split-K ta_gemm_h16sk_<tile> (as h16, k_splits
// workgroups per tile).
#define TA_GEMM_PIPE(NAME, BM, BN, BK, WGM, WGN, NS, C_F16, SPLIT, DBUF, DUAL)                \
  extern "C" __global__ __launch_bounds__(64 * WGM * WGN) void NAME(GemmArgs p) {             \
    static_assert(64 * WGM * WGN == ta_h16_lds_threads(BM, BN), "host launch width");         \
    GemmH16Pipe<BM, BN, BK, WGM, WGN, NS, C_F16, SPLIT, DBUF, DUAL>::run(p);                  \
  }
#define TA_GEMM_LDS(TAG, BM, BN, BK, WGM, WGN, NS, DBUF)                                      \
  TA_GEMM_PIPE(ta_gemm_h16_##TAG##_lds, BM, BN, BK, WGM, WGN, NS, false, false, DBUF, false)  \
  TA_GEMM_PIPE(ta_gemm_a16_##TAG##_lds, BM, BN, BK, WGM, WGN, NS, true, false, DBUF, false)
#define TA_GEMM_SK(TAG, BM, BN, BK, WGM, WGN, NS)                                             \
  TA_GEMM_PIPE(ta_gemm_h16sk_##TAG, BM, BN, BK, WGM, WGN, NS, false, true, true, false)
// SwiGLU pair in one pass: C = act(alpha * A @ B + bias) * U with
// U = alpha * A @ B2 stored to c2 (A read once for both weight matrices).
#define TA_GEMM_DUAL(TAG, BM, BN, BK, WGM, WGN, NS, DBUF)                                     \
  TA_GEMM_PIPE(ta_gemm_h16dual_##TAG##_lds, BM, BN, BK, WGM, WGN, NS, false, false, DBUF, true)

// Stage counts and loop forms as measured fastest on the config-5 shapes
// and 4096^3 (64 x 64: 11.9 us for 512x2048x2048; 128 x 64: 14.4 us for
// 512x2560x2048; 128 x 128: 21.7 us for 512x5632x2048; split 128 x 64,
// S = 2: 22.1 us for 512x2048x5632; 256 x 256: 110 us for 4096^3).  The
// 128 x 128 tiles run 16 waves.  The 64 x 64 tile reads each stage's
// fragments just before its MFMAs (one register set: O-proj 21.5 us
// against 22.1-22.6 us with two, timed with its conversion).  The dual
// 128 x 128 tile keeps one register set too (with two, its accumulator
// sets spill at 16 waves); the other three waves of each SIMD cover the
// reads, and the config-5 layer took 114.6 us against 120.4-121.4 us with
// 8 waves, 32-deep slabs through 5 stages and two fragment sets.
#ifndef TA_PIPE_TILES
TA_GEMM_LDS(m256n256, 256, 256, 64, 2, 4, 2, false)
TA_GEMM_LDS(m128n128, 128, 128, 64, 4, 4, 4, true)
TA_GEMM_LDS(m128n64, 128, 64, 64, 4, 2, 4, true)
TA_GEMM_LDS(m64n128, 64, 128, 64, 2, 4, 4, true)
TA_GEMM_LDS(m64n64, 64, 64, 64, 2, 2, 4, false)
TA_GEMM_SK(m64n128, 64, 128, 64, 2, 4, 4)
TA_GEMM_SK(m128n64, 128, 64, 64, 4, 2, 4)
TA_GEMM_SK(m128n128, 128, 128, 64, 4, 4, 4)
TA_GEMM_DUAL(m128n128, 128, 128, 64, 4, 4, 3, false)
TA_GEMM_DUAL(m128n64, 128, 64, 64, 4, 2, 4, true)
TA_GEMM_DUAL(m64n128, 64, 128, 64, 2, 4, 3, true)
TA_GEMM_DUAL(m64n64, 64, 64, 64, 2, 2, 4, true)
#else
TA_PIPE_TILES
#endif
// f32 -> f16 (RNE) of n elements, 8 per thread (block b of a launch):
// the A pre-pass of the pipelined f16w kernels.
namespace {
TA_DEVICE void cvt_block(const CvtArgs &p, uint64_t b) {
  const uint64_t i = (b * 256 + threadIdx.x) * 8;
  if (i + 8 <= p.n) {
    const f32x4 lo = *reinterpret_cast<const f32x4 *>(p.src + i);
    const f32x4 hi = *reinterpret_cast<const f32x4 *>(p.src + i + 4);
    f16x8 o;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      o[c] = (_Float16)lo[c];
      o[c + 4] = (_Float16)hi[c];
    }
    *reinterpret_cast<f16x8 *>(reinterpret_cast<_Float16 *>(p.dst) + i) = o;
  } else {
    for (uint64_t j = i; j < p.n; ++j)
      reinterpret_cast<_Float16 *>(p.dst)[j] = (_Float16)p.src[j];
  }
}
} // namespace

extern "C" __global__ __launch_bounds__(256) void ta_cvt_f32_f16(CvtArgs p) {
  cvt_block(p, blockIdx.x);
}

extern "C" __global__ __launch_bounds__(256) void ta_cvt_f32_f16_pair(CvtPairArgs p) {
  if (blockIdx.x < p.blocks0)
    cvt_block(p.job[0], blockIdx.x);
  else
    cvt_block(p.job[1], blockIdx.x - p.blocks0);
}
