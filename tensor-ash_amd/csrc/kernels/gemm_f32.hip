// FP32-MFMA GEMM with the fused epilogue, for gfx950 (CDNA4).
//
// Replaces the reference's SIMT f32 / f16w GEMM family
// (shaders/matmul_bda_v4_kernel.glsl:225-533 + matmul_epilogue_common.glsl)
// and its split-K stage 1 (shaders/matmul_splitk2_kernel.glsl:121-216).
// Same semantics: C = epilogue(alpha * A @ B (+C)), f32 accumulation, B in
// f32 or f16 storage (f16 widened exactly to f32 at LDS staging).
//
// Design (one workgroup per BM x BN output tile, 64-wide waves):
//  * v_mfma_f32_32x32x2_f32: each wave owns a (BM/WGM) x (BN/WGN) sub-tile
//    as FM x FN blocks of 32x32 accumulators (16 floats per lane per block).
//  * K is walked in slabs of BK = 16 (32 for the 256x256 tile), each
//    processed as 16-deep halves.  A slab of A is staged in LDS as
//    As[m][k] (k contiguous, +4 pad) so a lane reads its eight k values for
//    one slab with two 128-bit LDS reads; B is staged as Bs[k][n] (+4 pad)
//    and read 32 consecutive columns per half-wave.  The MFMA k index a lane
//    feeds at step s is (lane / 32) * 8 + s for both operands; any fixed
//    assignment of k to (lane group, step) sums the same products.
//  * Two LDS buffers plus one register stage: the global loads for slab
//    t+1 are issued before the MFMAs of slab t, written to the idle LDS
//    buffer after them, with one barrier per slab.
//  * Split-K stage 1 (num_splits > 1): grid.z = batch * splits; each split
//    masks its K window [k_lo, k_hi) at load time (zero fill), so the MFMA
//    loop is unchanged, and stores alpha * partial into its scratch plane.
//  * Ragged M/N/K: loads are zero-filled outside the matrix, stores are
//    guarded.  VEC kernels (K % 4 == 0 and N % 4 == 0) use 128-bit
//    (64-bit for f16 B) global loads; the others load scalars.
#include "common.h"

#include <utility>

namespace {

template <int BM, int BN, int WGM, int WGN, bool VEC, bool HALF_B, int BK_ = 16>
struct GemmF32 {
  static constexpr int BK = BK_;
  static constexpr int T = 64 * WGM * WGN;
  static constexpr int WTM = BM / WGM;
  static constexpr int WTN = BN / WGN;
  static constexpr int FM = WTM / 32;
  static constexpr int FN = WTN / 32;
  static constexpr int LDA = BK + 4;
  static constexpr int LDB = BN + 4;
  static constexpr int A_PER = BM * BK / 4 / T; // float4 units per thread
  static constexpr int B_PER = BK * BN / 4 / T;
  static constexpr int A_STAGE = BM * LDA;
  static constexpr int B_STAGE = BK * LDB;
  static_assert(A_PER * T * 4 == BM * BK, "A slab must split evenly");
  static_assert(B_PER * T * 4 == BK * BN, "B slab must split evenly");
  static_assert(FM >= 1 && FN >= 1, "wave tile must be a multiple of 32");
  static_assert(T / 64 * 32 * (WTN + 4) <= 2 * (A_STAGE + B_STAGE), "C staging fits in LDS");

  typedef typename std::conditional<HALF_B, const _Float16, const float>::type BT;

  // Global -> registers for one slab at absolute k offset k0, masking
  // rows >= M, cols >= N and k outside [klo, khi).
  static TA_DEVICE void load_a(const float *A, uint32_t M, uint32_t K,
                               uint32_t m0, uint32_t k0, uint32_t klo,
                               uint32_t khi, bool full, uint32_t tid,
                               f32x4 (&ra)[A_PER]) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const uint32_t e = tid + i * T;
      const uint32_t row = e / (BK / 4);
      const uint32_t kq = e % (BK / 4);
      const uint32_t gm = m0 + row;
      const uint32_t gk = k0 + kq * 4;
      const float *src = A + (uint64_t)gm * K + gk;
      if (VEC && full) {
        ra[i] = *reinterpret_cast<const f32x4 *>(src);
      } else if (full) {
        ra[i] = f32x4{src[0], src[1], src[2], src[3]};
      } else {
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (gm < M) {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (gk + c >= klo && gk + c < khi)
              v[c] = src[c];
        }
        ra[i] = v;
      }
    }
  }

  static TA_DEVICE void load_b(BT *B, uint32_t N, uint32_t n0, uint32_t k0,
                               uint32_t klo, uint32_t khi, bool full,
                               uint32_t tid, f32x4 (&rb)[B_PER]) {
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const uint32_t e = tid + i * T;
      const uint32_t kr = e / (BN / 4);
      const uint32_t nq = e % (BN / 4);
      const uint32_t gk = k0 + kr;
      const uint32_t gn = n0 + nq * 4;
      BT *src = B + (uint64_t)gk * N + gn;
      if (VEC && full) {
        if constexpr (HALF_B) {
          f16x4 h = *reinterpret_cast<const f16x4 *>(src);
          rb[i] = f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
        } else {
          rb[i] = *reinterpret_cast<const f32x4 *>(src);
        }
      } else if (full) {
        rb[i] = f32x4{(float)src[0], (float)src[1], (float)src[2], (float)src[3]};
      } else {
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (gk >= klo && gk < khi) {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (gn + c < N)
              v[c] = (float)src[c];
        }
        rb[i] = v;
      }
    }
  }

  static TA_DEVICE void store_lds(float *As, float *Bs, uint32_t tid,
                                  const f32x4 (&ra)[A_PER],
                                  const f32x4 (&rb)[B_PER]) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const uint32_t e = tid + i * T;
      *reinterpret_cast<f32x4 *>(&As[(e / (BK / 4)) * LDA + (e % (BK / 4)) * 4]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const uint32_t e = tid + i * T;
      *reinterpret_cast<f32x4 *>(&Bs[(e / (BN / 4)) * LDB + (e % (BN / 4)) * 4]) = rb[i];
    }
  }

  static TA_DEVICE void compute(const float *As, const float *Bs, uint32_t lane,
                                uint32_t wm, uint32_t wn,
                                f32x16 (&acc)[FM][FN]) {
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16)
      compute16(As + kk, Bs + kk * LDB, lane, wm, wn, acc);
  }

  // One 16-deep part of the slab (As / Bs offset to its first k).
  static TA_DEVICE void compute16(const float *As, const float *Bs, uint32_t lane,
                                  uint32_t wm, uint32_t wn,
                                  f32x16 (&acc)[FM][FN]) {
    const uint32_t lr = lane & 31u, lg = lane >> 5;
    float a[FM][8], b[FN][8];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const float *p = &As[(wm * WTM + fm * 32 + lr) * LDA + lg * 8];
      const f32x4 lo = *reinterpret_cast<const f32x4 *>(p);
      const f32x4 hi = *reinterpret_cast<const f32x4 *>(p + 4);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        a[fm][c] = lo[c];
        a[fm][c + 4] = hi[c];
      }
    }
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int s = 0; s < 8; ++s)
        b[fn][s] = Bs[(lg * 8 + s) * LDB + wn * WTN + fn * 32 + lr];
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
          acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[fm][s], b[fn][s],
                                                             acc[fm][fn], 0, 0, 0);
  }

  static TA_DEVICE void run(const GemmArgs &p) {
    __shared__ __attribute__((aligned(16))) float smem[2 * (A_STAGE + B_STAGE)];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t wm = wave / WGN, wn = wave % WGN;

    uint32_t tm, tn;
    ta_tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;

    const uint32_t P = p.num_splits;
    const uint32_t batch = blockIdx.z / P;
    const uint32_t split = blockIdx.z % P; // partial plane
    uint32_t klo = 0, khi = p.k;
    if (P > 1) {
      // Window of split s (shaders/matmul_splitk2_kernel.glsl:138-142),
      // then sub-window t of it by the same rule.
      const uint32_t T = max(1u, p.sub_splits), S = P / T;
      const uint32_t s = split / T, t = split % T;
      const uint32_t per = p.k / S, rem = p.k % S;
      const uint32_t lo = s * per + min(s, rem);
      const uint32_t len = per + (s < rem ? 1u : 0u);
      const uint32_t per2 = len / T, rem2 = len % T;
      klo = lo + t * per2 + min(t, rem2);
      khi = klo + per2 + (t < rem2 ? 1u : 0u);
    }

    const float *A = static_cast<const float *>(p.a) + (uint64_t)batch * p.stride_a;
    BT *B = static_cast<BT *>(p.b) + (uint64_t)batch * p.stride_b;
    const bool mn_full = (m0 + BM <= p.m) && (n0 + BN <= p.n);

    f32x16 acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          acc[fm][fn][r] = 0.0f;

    const uint32_t kt_lo = klo / BK;
    const uint32_t kt_hi = (khi + BK - 1) / BK;
    f32x4 ra[A_PER], rb[B_PER];

    if (kt_lo < kt_hi) {
      {
        const uint32_t k0 = kt_lo * BK;
        const bool full = mn_full && k0 >= klo && k0 + BK <= khi;
        load_a(A, p.m, p.k, m0, k0, klo, khi, full, tid, ra);
        load_b(B, p.n, n0, k0, klo, khi, full, tid, rb);
        store_lds(smem, smem + A_STAGE, tid, ra, rb);
      }
      __syncthreads();
      for (uint32_t kt = kt_lo; kt < kt_hi; ++kt) {
        const uint32_t cur = (kt - kt_lo) & 1u;
        float *As = smem + cur * (A_STAGE + B_STAGE);
        const bool more = kt + 1 < kt_hi;
        if (more) {
          const uint32_t k0 = (kt + 1) * BK;
          const bool full = mn_full && k0 >= klo && k0 + BK <= khi;
          load_a(A, p.m, p.k, m0, k0, klo, khi, full, tid, ra);
          load_b(B, p.n, n0, k0, klo, khi, full, tid, rb);
        }
        compute(As, As + A_STAGE, lane, wm, wn, acc);
        if (more) {
          float *Nx = smem + (cur ^ 1u) * (A_STAGE + B_STAGE);
          store_lds(Nx, Nx + A_STAGE, tid, ra, rb);
        }
        __syncthreads();
      }
    }

    ta_store_tile<WTM, WTN, FM, FN, T, false>(smem, 2 * (A_STAGE + B_STAGE), acc, p, lane, wave,
                                              wm, wn, m0, n0, batch, split);
  }
};


template <class F, int... I>
TA_DEVICE void ta_static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F> TA_DEVICE void ta_static_for(F &&f) {
  ta_static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Pipelined FP32 kernel for whole BM x BN tiles of f32 A and B whose
// K windows hold a multiple of 64 (K % (64 * splits) == 0): the shape of
// the fastest vendor FP32 kernels on this chip, written out by hand.  The
// 256x256 instance (2x2 waves of 128x128) serves plain GEMMs; 64x64 (2x2
// waves of 32x32) and 32x64 (1x2 waves of 32x32) serve split-K stage 1,
// 64x256 and 32x128 plain GEMMs that select those tiles,
// where grid.z = batch * splits and each split writes its partial tile.
//  * v_mfma_f32_16x16x4_f32; FM x FN blocks of 16x16 accumulators per wave
//    (256 registers per lane at 128x128, kept in the AGPRs).  MFMA step s
//    of a 16-deep stage takes k = (lane / 16) * 4 + s from both operands.
//  * NS stages (ta_mi16_stages: 8 for the 32x128 tile, whose two waves
//    per CU need the deeper look-ahead to cover the loaded memory latency,
//    and for the 64x64 split-K tile with its 8 KiB stages; 4 elsewhere,
//    where 8 measured slower) of 16-deep A [BM][16] and
//    B [16][BN] slabs in LDS,
//    filled by direct global -> LDS loads (global_load_lds_dwordx4) with
//    16-byte chunks XOR-swizzled per row on the global side:
//      A rows (64 bytes): chunk ^ ((b1 ^ b2) | (b2 ^ b3) << 1) of the row
//        index.  Chosen by measurement (SQ_LDS_BANK_CONFLICT): the pattern
//        chunk ^ ((b1 ^ b3) | b2 << 1), which separates 8 and 16
//        consecutive rows on paper, spent a quarter of the LDS's active
//        cycles on bank conflicts in every tile; this one none;
//      B rows (BN * 4 bytes): chunk ^ 4 * ((row >> 2) & 3), so the four rows a
//        wave reads at once (k = group * 4 + s) use four 16-bank quarters.
//  * One barrier per stage.  The LDS operands of stage k+1 are read into a
//    second register set while stage k's MFMAs run: the side operations of
//    a stage (direct loads, ds_read_b128 of A, ds_read2st64_b32 of B) go
//    one after each of its first MFMAs, so their latency is covered by the
//    rest of the stage and the MFMA pipe never waits on LDS.  The MFMAs and side
//    operations are volatile inline asm so this order is the one executed;
//    the explicit s_waitcnt at the end of a stage covers the register set
//    read during it.
//  * The side operations need no VALU work: direct loads address through a
//    wave-uniform 64-bit base advanced with scalar adds plus a fixed 32-bit
//    lane offset, and LDS reads use fixed base registers (one set per
//    stage pair) with the stage in the immediate offset.  Vector address
//    arithmetic between MFMAs measurably stalls the MFMA pipe.
//  * The loop is branch-free: K / 16 stages are walked four at a time (the
//    stage index, and so every LDS offset, is a compile-time constant in
//    each copy), and loads past the last stage re-read the last stage
//    (clamped source) into buffers nobody reads.
//  * Output through ta_store_tile_staged (the fused epilogue).
template <int BM, int BN, int WGM, int WGN, int NS> struct GemmF32Mi16 {
  static constexpr int BK = 16, T = 64 * WGM * WGN;
  static constexpr int WTM = BM / WGM, WTN = BN / WGN, FM = WTM / 16, FN = WTN / 16;
  static constexpr int A_BYTES = BM * BK * 4, B_BYTES = BK * BN * 4, STAGE = A_BYTES + B_BYTES;
  static constexpr int CPA = BK / 4, CPR = BN / 4; // 16-byte chunks per A / B row
  static constexpr int A_LD = A_BYTES / 16 / T, B_LD = B_BYTES / 16 / T, LD = A_LD + B_LD;
  static constexpr int SMEM_BYTES = NS * STAGE;
  static constexpr int READS = FM + 2 * FN; // LDS reads per stage
  static constexpr int MFMAS = 4 * FM * FN; // per stage
  static constexpr int SIDE = LD + READS;   // side operations per stage
  static constexpr int RU = BN / 64;        // a B row in 256-byte ds_read2st64 units
  static_assert(NS >= 4 && NS % 2 == 0, "the loop is unrolled by NS stages, NS / 2 LDS base groups");
  static_assert((NS - 3) * LD <= 63, "vmcnt range");
  static_assert(A_LD * T * 16 == A_BYTES && B_LD * T * 16 == B_BYTES, "stages split evenly");
  static_assert(SIDE <= MFMAS && 2 * LD <= SIDE, "side operations fit between the MFMAs");
  static_assert(CPA == 4 && CPR >= 16, "swizzles assume 64-byte A rows, >= 256-byte B rows");
  static_assert(WGM * WGN * 32 * (WTN + 4) * 4 <= SMEM_BYTES, "C staging fits in LDS");
  static_assert(STAGE % 256 == 0 && STAGE / 256 + 3 * RU <= 255, "ds_read2st64 offsets");
  typedef float f32x2 __attribute__((ext_vector_type(2)));

  static TA_DEVICE uint32_t swz_a(uint32_t row) {
    return ((row >> 1) ^ (row >> 2)) & 3u;
  }
  static TA_DEVICE uint32_t swz_b(uint32_t row) { return 4u * ((row >> 2) & 3u); }
  // The side operation issued after MFMA i of a stage, or -1: one after
  // each of the first SIDE MFMAs, so the next stage's LDS reads land under
  // this stage's remaining MFMAs.  (Spread evenly over the stage, the last
  // read followed the last MFMA and its latency was exposed at the stage's
  // closing lgkmcnt wait: 5% of a 64x64 split-K tile's stage-1 time, ~1%
  // of the 256x256 tile's.)
  static constexpr int side_after(int i) { return i < SIDE ? i : -1; }

  static TA_DEVICE void run(const GemmArgs &p) {
    __shared__ __attribute__((aligned(1024))) char smem[SMEM_BYTES];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave / WGN, wn = wave % WGN;
    const uint32_t P = p.num_splits;
    // Split-K with several tiles per window: consecutive dispatch ids go
    // to different XCDs, so deal (window, tile) pairs to the XCDs in
    // contiguous runs - the tiles of one K window then share its A rows in
    // one XCD's L2.  Which workgroup computes a plane does not change its
    // value.
    uint32_t bx = blockIdx.x, bz = blockIdx.z;
    {
      const uint32_t tiles = gridDim.x, G = tiles * gridDim.z;
      if (P > 1 && tiles > 1 && G % (8 * tiles) == 0) {
        const uint32_t L = bz * tiles + bx, v = (L & 7u) * (G >> 3) + (L >> 3);
        bz = v / tiles;
        bx = v % tiles;
      }
    }
    uint32_t tm, tn;
    ta_tile_coords(bx, p.tiles_m, p.tiles_n, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t batch = bz / P, split = bz % P;
    // Split-K window (the GemmF32 rule; the host sends only shapes whose
    // windows all hold a multiple of 64 rows of K).
    uint32_t klo = 0, khi = p.k;
    if (P > 1) {
      const uint32_t Tt = max(1u, p.sub_splits), S = P / Tt;
      const uint32_t sp = split / Tt, t = split % Tt;
      const uint32_t per = p.k / S, rem = p.k % S;
      const uint32_t lo = sp * per + min(sp, rem);
      const uint32_t len = per + (sp < rem ? 1u : 0u);
      const uint32_t per2 = len / Tt, rem2 = len % Tt;
      klo = lo + t * per2 + min(t, rem2);
      khi = klo + per2 + (t < rem2 ? 1u : 0u);
    }
    const float *A = static_cast<const float *>(p.a) + (uint64_t)batch * p.stride_a + klo;
    const float *B = static_cast<const float *>(p.b) + (uint64_t)batch * p.stride_b +
                     (uint64_t)klo * p.n;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)smem;
    const uint32_t kts = (khi - klo) / BK;

    // Direct loads: wave-uniform 64-bit base (per stage) + per-lane 32-bit offset.
    uint32_t avoff[A_LD], bvoff[B_LD];
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const uint32_t q = i * T + tid, row = q / CPA, c = (q % CPA) ^ swz_a(row);
      avoff[i] = row * p.k * 4 + 16 * c;
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const uint32_t q = i * T + tid, row = q / CPR, c = (q % CPR) ^ swz_b(row);
      bvoff[i] = row * p.n * 4 + 16 * c;
    }
    const char *abase0 = reinterpret_cast<const char *>(A + (uint64_t)m0 * p.k);
    const char *bbase0 = reinterpret_cast<const char *>(B + n0);
    const uint64_t b_stage = (uint64_t)BK * p.n * 4;
    const uint32_t lr = lane & 15u, lg = lane >> 4;
    // LDS read bases for stage pairs {2g, 2g + 1} (group g); the stage
    // within a group is the instruction's immediate offset.
    uint32_t a_off[NS / 2][FM], b_off[NS / 2][FN];
#pragma unroll
    for (int g = 0; g < NS / 2; ++g) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const uint32_t row = wm * WTM + fm * 16 + lr;
        a_off[g][fm] = lds0 + g * 2 * STAGE + row * (BK * 4) + 16u * (lg ^ swz_a(row));
      }
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const uint32_t col = wn * WTN + fn * 16 + lr, row = lg * 4u;
        b_off[g][fn] = lds0 + g * 2 * STAGE + A_BYTES + row * (BN * 4) +
                       16u * ((col >> 2) ^ swz_b(row)) + (col & 3u) * 4;
      }
    }
    f32x4 acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
        acc[fm][fn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 ra[2][FM];
    f32x2 rb[2][FN][2];

    // i-th direct load of stage j (A chunks first, then B); loads past the
    // last stage re-read it into a buffer nobody reads.
    auto gload = [&](uint32_t j, auto i_c) __attribute__((always_inline)) {
      constexpr int i = decltype(i_c)::value;
      const uint32_t jj = min(j, kts - 1u);
      const uint32_t base = lds0 + (j % NS) * STAGE + wave * 64 * 16;
      if constexpr (i < A_LD) {
        const char *sb = abase0 + (uint64_t)jj * BK * 4;
        const uint32_t vo = avoff[i];
        asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(vo), "s"(sb),
                     "s"(base + i * T * 16) : "memory", "m0");
      } else {
        const char *sb = bbase0 + (uint64_t)jj * b_stage;
        const uint32_t vo = bvoff[i - A_LD];
        asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(vo),
                     "s"(sb), "s"(base + A_BYTES + (i - A_LD) * T * 16) : "memory", "m0");
      }
    };
    // i-th LDS read of stage `stg` (compile time) into register set `set`.
    auto lread = [&](auto set_c, auto stg_c, auto i_c) __attribute__((always_inline)) {
      constexpr int set = decltype(set_c)::value, stg = decltype(stg_c)::value, i = decltype(i_c)::value;
      constexpr int g = stg / 2, so = (stg % 2) * STAGE;
      if constexpr (i < FM) {
        f32x4 v;
        const uint32_t ad = a_off[g][i];
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(ad), "n"(so) : "memory");
        ra[set][i] = v;
      } else {
        constexpr int fn = (i - FM) / 2, h = (i - FM) % 2;
        // rows group * 4 + 2h and + 1 of the B slab
        constexpr int o0 = so / 256 + 2 * RU * h, o1 = o0 + RU;
        const uint32_t bd = b_off[g][fn];
        f32x2 v;
        asm volatile("ds_read2st64_b32 %0, %1 offset0:%2 offset1:%3"
                     : "=v"(v) : "v"(bd), "n"(o0), "n"(o1) : "memory");
        rb[set][fn][h] = v;
      }
    };
    auto mfma = [&](auto set_c, auto idx_c) __attribute__((always_inline)) {
      constexpr int set = decltype(set_c)::value, idx = decltype(idx_c)::value;
      constexpr int s = idx / (FM * FN), fm = (idx / FN) % FM, fn = idx % FN;
      f32x4 c = acc[fm][fn];
      const float av = ra[set][fm][s], bv = rb[set][fn][s / 2][s % 2];
      asm volatile("v_mfma_f32_16x16x4_f32 %0, %1, %2, %0" : "+a"(c) : "v"(av), "v"(bv));
      acc[fm][fn] = c;
    };

    for (uint32_t j = 0; j < NS - 1; ++j)
      ta_static_for<LD>([&](auto i_c) __attribute__((always_inline)) { gload(j, i_c); });
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NS - 2) * LD) : "memory");
    __syncthreads();
    ta_static_for<READS>([&](auto i_c) __attribute__((always_inline)) {
      lread(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, i_c);
    });
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    // Stage kt: MFMAs on register set `cur`; loads of stage kt + NS - 1
    // and LDS reads of stage kt + 1 (into the other set) in between.
    auto body = [&](auto stg_c, uint32_t kt) __attribute__((always_inline)) {
      constexpr int stg = decltype(stg_c)::value, cur = stg % 2; // stg = kt % NS
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NS - 3) * LD) : "memory");
      // Side operation j follows MFMA j: loads at the even slots below
      // 2 * LD, LDS reads in the others.
      ta_static_for<MFMAS>([&](auto ic) __attribute__((always_inline)) {
        constexpr int i = decltype(ic)::value;
        mfma(std::integral_constant<int, cur>{}, ic);
        constexpr int side = side_after(i);
        if constexpr (side >= 0) {
          if constexpr (side < 2 * LD && (side & 1) == 0)
            gload(kt + NS - 1, std::integral_constant<int, side / 2>{});
          else
            lread(std::integral_constant<int, 1 - cur>{}, std::integral_constant<int, (stg + 1) % NS>{},
                  std::integral_constant<int, (side < 2 * LD ? side / 2 : side - LD)>{});
        }
      });
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    };
    for (uint32_t kt = 0; kt < kts; kt += NS) {
      ta_static_for<NS>([&](auto sc) __attribute__((always_inline)) {
        body(sc, kt + decltype(sc)::value);
      });
      // The MFMAs are inline asm, so the compiler does not know their result
      // latency: wait states after each iteration's last MFMAs, so copies
      // the compiler places at the loop exit read settled accumulators.
      asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
    }
    // Drain the trailing loads (they re-read the last stage into buffers
    // nobody reads) before the LDS is reused for the write-out.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    // 16x16 blocks: lane l holds rows 4*(l/16) + i, column l%16.
    constexpr int LDC = WTN + 4;
    auto stage = [&](float *Cs, int blk) __attribute__((always_inline)) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        if (fm / 2 != blk)
          continue;
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            Cs[((fm % 2) * 16 + 4 * lg + i) * LDC + fn * 16 + lr] = acc[fm][fn][i];
      }
    };
    ta_store_tile_staged<WTM, WTN, T, false>(reinterpret_cast<float *>(smem), stage, p, lane, wave,
                                             wm, wn, m0, n0, batch, split);
  }
};

} // namespace

#define TA_GEMM_F32(NAME, BM, BN, WGM, WGN, VEC, HALF_B, BK)                      \
  extern "C" __global__ __launch_bounds__(64 * WGM * WGN) void NAME(GemmArgs p) { \
    GemmF32<BM, BN, WGM, WGN, VEC, HALF_B, BK>::run(p);                          \
  }

#define TA_GEMM_F32_FAMILY(TAG, BM, BN, WGM, WGN, BK)                           \
  TA_GEMM_F32(ta_gemm_f32_##TAG##_vec, BM, BN, WGM, WGN, true, false, BK)       \
  TA_GEMM_F32(ta_gemm_f32_##TAG##_gen, BM, BN, WGM, WGN, false, false, BK)      \
  TA_GEMM_F32(ta_gemm_f16w_##TAG##_vec, BM, BN, WGM, WGN, true, true, BK)       \
  TA_GEMM_F32(ta_gemm_f16w_##TAG##_gen, BM, BN, WGM, WGN, false, true, BK)

// The 256x256 tile walks K in 32-deep slabs (half the barriers; its two
// 70 KiB LDS buffers still fit), the others in 16-deep slabs.
TA_GEMM_F32_FAMILY(m256n256, 256, 256, 2, 4, 32)
TA_GEMM_F32_FAMILY(m256n128, 256, 128, 2, 2, 16)
TA_GEMM_F32_FAMILY(m128n128, 128, 128, 2, 2, 16)
TA_GEMM_F32_FAMILY(m128n64, 128, 64, 2, 2, 16)
TA_GEMM_F32_FAMILY(m64n64, 64, 64, 2, 2, 16)
// Skinny tiles (whole N of a deep-K split-K stage 1 in one tile, so A is
// read once): 64x256 with 1x4 waves, 32x128 with 1x2 waves (128 threads).
TA_GEMM_F32_FAMILY(m64n256, 64, 256, 1, 4, 16)
TA_GEMM_F32_FAMILY(m32n128, 32, 128, 1, 2, 16)
TA_GEMM_F32_FAMILY(m32n64, 32, 64, 1, 2, 16)

// Whole tiles of f32 A and B whose K windows hold multiples of 64 rows
// (see GemmF32Mi16): the 256x256 data-parallel tile and the split-K
// stage-1 tiles (64x64 and 32x64: several column tiles per K window, so
// the windows are longer and the partial planes fewer than with one tile
// spanning N).
extern "C" __global__ __launch_bounds__(256) void ta_gemm_f32_m256n256_mi16(GemmArgs p) {
  GemmF32Mi16<256, 256, 2, 2, ta_mi16_stages(256, 256)>::run(p);
}
extern "C" __global__ __launch_bounds__(256) void ta_gemm_f32_m64n256_mi16(GemmArgs p) {
  GemmF32Mi16<64, 256, 1, 4, ta_mi16_stages(64, 256)>::run(p);
}
extern "C" __global__ __launch_bounds__(128) void ta_gemm_f32_m32n128_mi16(GemmArgs p) {
  GemmF32Mi16<32, 128, 1, 2, ta_mi16_stages(32, 128)>::run(p);
}
extern "C" __global__ __launch_bounds__(256) void ta_gemm_f32_m64n64_mi16(GemmArgs p) {
  GemmF32Mi16<64, 64, 2, 2, ta_mi16_stages(64, 64)>::run(p);
}
extern "C" __global__ __launch_bounds__(128) void ta_gemm_f32_m32n64_mi16(GemmArgs p) {
  GemmF32Mi16<32, 64, 1, 2, ta_mi16_stages(32, 64)>::run(p);
}
