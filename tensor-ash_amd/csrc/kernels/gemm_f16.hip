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
