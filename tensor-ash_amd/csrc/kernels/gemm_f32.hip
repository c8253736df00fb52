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

