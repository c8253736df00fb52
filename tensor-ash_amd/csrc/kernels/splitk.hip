// Stage 2 of the deterministic two-stage split-K (stage 1 is the GEMM
// kernel with num_splits > 1, see gemm_f32.hip).
//
// Same contract as the reference's reduce
// (shaders/matmul_f32_splitk2_reduce.comp:44-75): for every output element
// e of batch b, C[b][e] = sum over s = 0..S-1, in that order, of
// scratch[(b * S + s) * mn + e].  No atomics anywhere, so the result is
// bit-identical from run to run for a fixed S.
//
// HBM-bound: it reads S planes once and writes one.  Each thread owns four
// consecutive elements (one 128-bit load per plane) when mn % 4 == 0, else
// four scalar elements; a grid-stride loop keeps the grid at a few waves
// per CU.
#include "common.h"

extern "C" __global__ __launch_bounds__(256) void ta_splitk_reduce(SplitReduceArgs p) {
  const uint64_t quads = (p.total + 3) / 4;
  const bool vec = (p.mn & 3u) == 0u;
  for (uint64_t q = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; q < quads;
       q += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t base = q * 4;
    if (vec) {
      const uint64_t b = base / p.mn, e = base % p.mn;
      const float *src = p.scratch + b * p.num_splits * p.mn + e;
      f32x4 acc = *reinterpret_cast<const f32x4 *>(src);
      for (uint32_t s = 1; s < p.num_splits; ++s)
        acc += *reinterpret_cast<const f32x4 *>(src + (uint64_t)s * p.mn);
      *reinterpret_cast<f32x4 *>(p.c + base) = acc;
    } else {
      for (uint32_t lane = 0; lane < 4; ++lane) {
        const uint64_t i = base + lane;
        if (i >= p.total)
          break;
        const uint64_t b = i / p.mn, e = i % p.mn;
        const float *src = p.scratch + b * p.num_splits * p.mn + e;
        float acc = src[0];
        for (uint32_t s = 1; s < p.num_splits; ++s)
          acc += src[(uint64_t)s * p.mn];
        p.c[i] = acc;
      }
    }
  }
}
