// Stage 2 of the deterministic two-stage split-K (stage 1 is the GEMM
// kernel with num_splits > 1, see gemm_f32.hip), which also applies the
// op's fused epilogue once, to the finished sum
// (shaders/matmul_epilogue_common.glsl:30-82 on the reduced value).
//
// Contract (the reference's reduce, shaders/matmul_f32_splitk2_reduce.comp:
// 44-75, sums the S planes of batch b in order; here there are P planes,
// S splits of P / S windows each): the P planes of batch b are cut into
// G = `groups` contiguous groups by the split-window rule; each group is
// summed in plane order, then the group sums are added pairwise in a fixed
// tree (g0 + g1, g2 + g3, ..., then those pairs, ...).
// The host derives G from the shape alone (enough threads to cover the
// chip), and nothing here uses atomics, so the result is bit-identical
// from run to run for a fixed shape and P.
//
// HBM-bound: it reads every plane once and writes one.  A workgroup of
// 256 threads owns 256 / G quads (four consecutive elements, one 128-bit
// load per plane when mn % 4 == 0); thread (g, quad) sums group g of its
// quad with up to 8 plane loads in flight ahead of the in-order adds, and
// the G group sums meet in LDS for the tree.
#include "common.h"

namespace {
constexpr int kThreads = 256, kBatch = 8;

// Quad starting at element `base` of plane `plane`; `off0` is its offset
// in plane 0 of its batch (vector path only: mn % 4 == 0 keeps a quad in
// one batch).
TA_DEVICE f32x4 load_quad(const SplitReduceArgs &p, bool vec, uint64_t base, uint64_t off0,
                          uint32_t plane) {
  if (vec)
    return *reinterpret_cast<const f32x4 *>(p.scratch + off0 + (uint64_t)plane * p.mn);
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
// The fused epilogue on the plane sum v of element i (batch-major index
// into C): the order of ta_epilogue with alpha already in v
// (shaders/matmul_epilogue_common.glsl:14-21).  A C read for accumulate
// happens before this thread's store of the same element.
TA_DEVICE float reduce_epilogue(const SplitReduceArgs &p, float v, uint64_t i) {
  if (p.flags & TA_FLAG_ACCUMULATE)
    v += p.c[i];
  if (p.flags & TA_FLAG_BIAS) {
    const uint32_t b = (uint32_t)(i / p.mn);
    const uint32_t col = (uint32_t)(i % p.mn % p.n);
    v += p.bias[(uint64_t)b * p.bias_batch_stride + col];
  }
  v = ta_activate(v, p.act);
  if (p.binary == TA_BIN_ADD_SCALED)
    v = fmaf(p.beta, p.d[i], v);
  else if (p.binary == TA_BIN_MUL)
    v *= p.d[i];
  return v;
}
} // namespace

extern "C" __global__ __launch_bounds__(kThreads) void ta_splitk_reduce(SplitReduceArgs p) {
  __shared__ f32x4 part[kThreads];
  const bool epi = p.flags != 0u || p.act != TA_ACT_NONE || p.binary != TA_BIN_NONE;
  const uint64_t quads = (p.total + 3) / 4;
  const bool vec = (p.mn & 3u) == 0u;
  const uint32_t P = p.num_splits;
  const uint32_t G = p.groups; // power of two <= min(P, 256), host-checked
  const uint32_t QW = kThreads / G; // quads per workgroup pass
  const uint32_t g = threadIdx.x / QW, ql = threadIdx.x % QW;
  const uint32_t per = P / G, rem = P % G;
  const uint32_t lo = g * per + min(g, rem);
  const uint32_t hi = lo + per + (g < rem ? 1u : 0u);
  for (uint64_t qb = blockIdx.x; qb * QW < quads; qb += gridDim.x) {
    const uint64_t q = qb * QW + ql;
    if (q < quads) {
      // Planes lo..hi-1 in order, loaded kBatch at a time ahead of their
      // adds so the loads overlap (one round trip when hi - lo <= kBatch);
      // the adds keep the plane order.
      const uint64_t base = q * 4;
      const uint64_t off0 = vec ? (base / p.mn) * P * p.mn + base % p.mn : 0;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      for (uint32_t s0 = lo; s0 < hi; s0 += kBatch) {
        f32x4 v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
          v[j] = s0 + j < hi ? load_quad(p, vec, base, off0, s0 + j) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
          if (s0 + j < hi)
            acc = s0 + j == lo ? v[j] : acc + v[j];
      }
      part[g * QW + ql] = acc;
    }
    // Group sums: fixed pairwise tree ((g0 + g1) + (g2 + g3)) + ...
    for (uint32_t step = 1; step < G; step *= 2) {
      __syncthreads();
      if ((g & (2 * step - 1)) == 0 && q < quads)
        part[g * QW + ql] += part[(g + step) * QW + ql];
    }
    __syncthreads();
    if (g == 0 && q < quads) {
      f32x4 r = part[ql];
      const uint64_t base = q * 4;
      if (epi)
        for (uint32_t c = 0; c < 4; ++c)
          if (base + c < p.total)
            r[c] = reduce_epilogue(p, r[c], base + c);
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
