// Stage 2 of the deterministic two-stage split-K (stage 1 is the GEMM
// kernel with num_splits > 1, see gemm_f32.hip).
//
// Contract (the reference's reduce, shaders/matmul_f32_splitk2_reduce.comp:
// 44-75, sums the S planes of batch b in order; here there are P planes,
// S splits of P / S windows each): the P planes of batch b are cut into
// G = min(P, 8) contiguous groups by the split-window rule; each group is
// summed in plane order, then the group sums are added in group order.
// No atomics anywhere, so the result is bit-identical from run to run for
// a fixed P.
//
// HBM-bound: it reads every plane once and writes one.  A workgroup owns
// 32 quads (four consecutive elements, one 128-bit load per plane when
// mn % 4 == 0) and spreads the G groups over its threads, so the plane
// loads of all groups are in flight together; group sums meet in LDS.
#include "common.h"

namespace {
constexpr int kGroups = 8, kQuads = 32;

TA_DEVICE f32x4 load_quad(const SplitReduceArgs &p, bool vec, uint64_t base, uint32_t plane) {
  if (vec) {
    const uint64_t b = base / p.mn, e = base % p.mn;
    return *reinterpret_cast<const f32x4 *>(p.scratch + (b * p.num_splits + plane) * p.mn + e);
  }
  f32x4 v = {0.f, 0.f, 0.f, 0.f};
  for (uint32_t c = 0; c < 4; ++c) {
    const uint64_t i = base + c;
    if (i < p.total) {
      const uint64_t b = i / p.mn, e = i % p.mn;
      v[c] = p.scratch[(b * p.num_splits + plane) * p.mn + e];
    }
  }
  return v;
}
} // namespace

extern "C" __global__ __launch_bounds__(256) void ta_splitk_reduce(SplitReduceArgs p) {
  __shared__ f32x4 part[kGroups][kQuads];
  const uint64_t quads = (p.total + 3) / 4;
  const bool vec = (p.mn & 3u) == 0u;
  const uint32_t P = p.num_splits;
  const uint32_t G = min((uint32_t)kGroups, P);
  const uint32_t g = threadIdx.x / kQuads, ql = threadIdx.x % kQuads;
  const uint32_t per = P / G, rem = P % G;
  const uint32_t lo = g * per + min(g, rem);
  const uint32_t hi = g < G ? lo + per + (g < rem ? 1u : 0u) : lo;
  for (uint64_t qb = blockIdx.x; qb * kQuads < quads; qb += gridDim.x) {
    const uint64_t q = qb * kQuads + ql;
    if (q < quads && lo < hi) {
      const uint64_t base = q * 4;
      f32x4 acc = load_quad(p, vec, base, lo);
      for (uint32_t s = lo + 1; s < hi; ++s)
        acc += load_quad(p, vec, base, s);
      part[g][ql] = acc;
    }
    __syncthreads();
    if (g == 0 && q < quads) {
      f32x4 r = part[0][ql];
      for (uint32_t gg = 1; gg < G; ++gg)
        r += part[gg][ql];
      const uint64_t base = q * 4;
      if (vec) {
        *reinterpret_cast<f32x4 *>(p.c + base) = r;
      } else {
        for (uint32_t c = 0; c < 4; ++c)
          if (base + c < p.total)
            p.c[base + c] = r[c];
      }
    }
    __syncthreads();
  }
}
