// The decode token loop on the GPU for gfx950: greedy argmax over the
// logits, the embedding-row gather that feeds the chosen token back as
// the next input, and split-K decode attention over the KV caches (the
// reference's op_argmax_f32.comp, op_embed_gather.comp and
// attention_decode_kernel.glsl + op_attn_decode_combine.comp; host side
// src/executor/elementwise/ops.rs:456-595 and attn.rs:14-185).
//
//  * argmax: one workgroup of 16 waves; each thread scans its elements in
//    ascending index order (128-bit loads when the input is 16-byte
//    aligned), then (value, index) pairs meet in a lexicographic max
//    (greater value, then greater index) across lanes and waves.  That
//    max does not depend on how the elements are split, so the result is
//    exactly "the last maximum" of the whole vector, as the reference's
//    greedy sampler defines it (Rust `max_by(total_cmp)` on finite data).
//  * gather: one thread per four columns of an output row, the token id
//    read on the device and clamped to vocab - 1.
//  * decode attention, stage 1: workgroup (chunk, kv head), 4 waves that
//    take 64-position blocks of the chunk in turn.  Per block, lane =
//    position for the scores (K^T rows are contiguous along positions,
//    one 256-byte wave load per head dimension), a wave max per query row
//    sets the block's running maximum, the probabilities go to LDS, and
//    lane = head dimension for P @ V (V rows are contiguous along dh).
//    Softmax runs in base 2 (scale folded with log2(e)); the stored max is
//    in log2 units, which stage 2 undoes with exp2.  Positions at or past
//    the chunk end are never read.  The four waves' states merge exactly
//    in LDS.
//  * stage 2: per (kv head, row), the chunks merge exactly:
//    m* = max m_i, w_i = 2^(m_i - m*), out = sum acc_i w_i / sum l_i w_i.
#include "common.h"

#include <float.h>

namespace {

constexpr uint32_t kArgmaxThreads = 1024;
constexpr uint32_t kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr int kAttnRows = 8; // query rows per kv head (GQA group), at most

TA_DEVICE void argmax_merge(float &v, uint32_t &i, float ov, uint32_t oi) {
  if (ov > v || (ov == v && oi > i)) {
    v = ov;
    i = oi;
  }
}

TA_DEVICE float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
    v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
TA_DEVICE float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
    v += __shfl_xor(v, o);
  return v;
}

// Orders this wave's LDS accesses before and after (lanes of one wave read
// what other lanes of the same wave wrote).
TA_DEVICE void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <bool KV16> TA_DEVICE float load_kv(const void *p, uint64_t i) {
  if constexpr (KV16)
    return (float)static_cast<const _Float16 *>(p)[i];
  else
    return static_cast<const float *>(p)[i];
}

template <int DH, bool KV16> struct AttnDecode {
  static constexpr int DPL = DH / 64; // head dimensions per lane in P @ V
  static constexpr int KU = 16;       // K^T loads in flight per group
  struct Smem {
    f32x4 qT[DH][kAttnRows / 4];             // q transposed: [d][row]
    f32x4 P[kAttnWaves][64][kAttnRows / 4];  // block probabilities: [pos][row]
    float mrg[kAttnWaves][kAttnRows][DH + 2]; // wave states: acc, m, l
  };

  static TA_DEVICE void run(const AttnDecodeArgs &p) {
    __shared__ Smem sm;
    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t group = p.group;
    float *qT = reinterpret_cast<float *>(sm.qT);
    for (uint32_t i = tid; i < DH * kAttnRows; i += kAttnThreads) {
      const uint32_t d = i / kAttnRows, r = i % kAttnRows;
      qT[i] = r < group ? p.q[((uint64_t)kvh * group + r) * DH + d] : 0.0f;
    }
    const uint32_t len = min(p.t_max, p.kv_len + (p.pos ? *p.pos : 0u));
    const uint32_t cs = (len + p.num_chunks - 1) / p.num_chunks;
    const uint32_t p0 = min(chunk * cs, len), p1 = min(p0 + cs, len);
    const float scale2 = p.scale * 1.4426950408889634f;
    const uint64_t kt_base = (uint64_t)kvh * DH * p.t_max;
    const uint64_t v_base = (uint64_t)kvh * p.t_max * DH;
    __syncthreads();

    float m[kAttnRows], lp[kAttnRows], acc[kAttnRows][DPL];
#pragma unroll
    for (int r = 0; r < kAttnRows; ++r) {
      m[r] = -FLT_MAX;
      lp[r] = 0.0f;
#pragma unroll
      for (int c = 0; c < DPL; ++c)
        acc[r][c] = 0.0f;
    }

    for (uint32_t blk = p0 + wave * 64; blk < p1; blk += kAttnWaves * 64) {
      const uint32_t pos = blk + lane;
      const bool valid = pos < p1;
      const uint64_t kcol = kt_base + (valid ? pos : blk);
      // Scores of this lane's position for every row.
      float s[kAttnRows];
#pragma unroll
      for (int r = 0; r < kAttnRows; ++r)
        s[r] = 0.0f;
#pragma unroll
      for (int d0 = 0; d0 < DH; d0 += KU) {
        float k[KU];
#pragma unroll
        for (int u = 0; u < KU; ++u)
          k[u] = load_kv<KV16>(p.kt, kcol + (uint64_t)(d0 + u) * p.t_max);
#pragma unroll
        for (int u = 0; u < KU; ++u) {
          const f32x4 qa = sm.qT[d0 + u][0], qb = sm.qT[d0 + u][1];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            s[r] = fmaf(qa[r], k[u], s[r]);
            s[r + 4] = fmaf(qb[r], k[u], s[r + 4]);
          }
        }
      }
      // Online softmax over the block: one running max per row (uniform
      // over the wave), per-lane partial sums rescaled with it.
      float e[kAttnRows];
#pragma unroll
      for (int r = 0; r < kAttnRows; ++r) {
        const float s2 = valid ? s[r] * scale2 : -INFINITY;
        const float mn = fmaxf(m[r], wave_max(s2));
        const float corr = exp2f(m[r] - mn);
        e[r] = exp2f(s2 - mn);
        lp[r] = fmaf(lp[r], corr, e[r]);
#pragma unroll
        for (int c = 0; c < DPL; ++c)
          acc[r][c] *= corr;
        m[r] = mn;
      }
      sm.P[wave][lane][0] = f32x4{e[0], e[1], e[2], e[3]};
      sm.P[wave][lane][1] = f32x4{e[4], e[5], e[6], e[7]};
      wave_lds_sync();
      // P @ V: lane = head dimension.
      const uint32_t nv = min(64u, p1 - blk);
      const uint64_t vrow = v_base + (uint64_t)blk * DH + lane;
      for (uint32_t j = 0; j < nv; ++j) {
        float vv[DPL];
#pragma unroll
        for (int c = 0; c < DPL; ++c)
          vv[c] = load_kv<KV16>(p.v, vrow + (uint64_t)j * DH + 64 * c);
        const f32x4 pa = sm.P[wave][j][0], pb = sm.P[wave][j][1];
#pragma unroll
        for (int c = 0; c < DPL; ++c)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            acc[r][c] = fmaf(pa[r], vv[c], acc[r][c]);
            acc[r + 4][c] = fmaf(pb[r], vv[c], acc[r + 4][c]);
          }
      }
      wave_lds_sync(); // P is rewritten by the next block
    }

    // Merge the four waves' states (an idle wave holds the identity).
#pragma unroll
    for (int r = 0; r < kAttnRows; ++r) {
      const float l = wave_sum(lp[r]);
#pragma unroll
      for (int c = 0; c < DPL; ++c)
        sm.mrg[wave][r][lane + 64 * c] = acc[r][c];
      if (lane == 0) {
        sm.mrg[wave][r][DH] = m[r];
        sm.mrg[wave][r][DH + 1] = l;
      }
    }
    __syncthreads();
    for (uint32_t i = tid; i < group * (DH + 2); i += kAttnThreads) {
      const uint32_t r = i / (DH + 2), d = i % (DH + 2);
      float ms = sm.mrg[0][r][DH];
#pragma unroll
      for (int w = 1; w < kAttnWaves; ++w)
        ms = fmaxf(ms, sm.mrg[w][r][DH]);
      float v;
      if (d == DH) {
        v = ms;
      } else {
        v = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w)
          v = fmaf(sm.mrg[w][r][d], exp2f(sm.mrg[w][r][DH] - ms), v);
      }
      p.scratch[(((uint64_t)kvh * p.num_chunks + chunk) * group + r) * (DH + 2) + d] = v;
    }
  }
};

} // namespace

extern "C" __global__ __launch_bounds__(kArgmaxThreads) void ta_argmax_f32(ArgmaxArgs p) {
  __shared__ float sv[kArgmaxThreads / 64];
  __shared__ uint32_t si[kArgmaxThreads / 64];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  float best = -INFINITY;
  uint32_t bi = 0;
  // Ascending per thread: its quads, then its tail elements (all past the
  // quads), so ">=" keeps the thread's last maximum.
  const uint32_t nq = (reinterpret_cast<uintptr_t>(p.in) & 15u) == 0 ? p.n / 4 : 0;
  for (uint32_t q = tid; q < nq; q += kArgmaxThreads) {
    const f32x4 v = reinterpret_cast<const f32x4 *>(p.in)[q];
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (v[c] >= best) {
        best = v[c];
        bi = 4 * q + c;
      }
  }
  for (uint32_t i = 4 * nq + tid; i < p.n; i += kArgmaxThreads) {
    const float v = p.in[i];
    if (v >= best) {
      best = v;
      bi = i;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
    argmax_merge(best, bi, __shfl_xor(best, o), __shfl_xor(bi, o));
  if (lane == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (wave == 0) {
    constexpr uint32_t W = kArgmaxThreads / 64;
    best = lane < W ? sv[lane] : -INFINITY;
    bi = lane < W ? si[lane] : 0u;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
      argmax_merge(best, bi, __shfl_xor(best, o), __shfl_xor(bi, o));
    if (lane == 0)
      *p.result = bi;
  }
}

extern "C" __global__ __launch_bounds__(256) void ta_embed_gather(EmbedArgs p) {
  const uint32_t t = blockIdx.y;
  const uint32_t i = (blockIdx.x * 256u + threadIdx.x) * 4u;
  if (t >= p.n_tokens || i >= p.embd)
    return;
  const uint32_t tok = min(p.tokens[t], p.vocab - 1u);
  const uint64_t src = (uint64_t)tok * p.embd + i, dst = (uint64_t)t * p.embd + i;
  if ((p.embd & 3u) == 0u) {
    const f32x4 v = p.table_f16
                        ? __builtin_convertvector(
                              *reinterpret_cast<const f16x4 *>(
                                  static_cast<const _Float16 *>(p.table) + src),
                              f32x4)
                        : *reinterpret_cast<const f32x4 *>(static_cast<const float *>(p.table) + src);
    if (p.out_f16)
      *reinterpret_cast<f16x4 *>(static_cast<_Float16 *>(p.out) + dst) =
          __builtin_convertvector(v, f16x4);
    else
      *reinterpret_cast<f32x4 *>(static_cast<float *>(p.out) + dst) = v;
    return;
  }
  for (uint32_t c = 0; c < 4 && i + c < p.embd; ++c) {
    const float v = p.table_f16 ? (float)static_cast<const _Float16 *>(p.table)[src + c]
                                : static_cast<const float *>(p.table)[src + c];
    if (p.out_f16)
      static_cast<_Float16 *>(p.out)[dst + c] = (_Float16)v;
    else
      static_cast<float *>(p.out)[dst + c] = v;
  }
}

#define TA_ATTN_DECODE(NAME, DH, KV16)                                                 \
  extern "C" __global__ __launch_bounds__(kAttnThreads) void NAME(AttnDecodeArgs p) { \
    AttnDecode<DH, KV16>::run(p);                                                      \
  }
TA_ATTN_DECODE(ta_attn_decode_dh64, 64, false)
TA_ATTN_DECODE(ta_attn_decode_dh128, 128, false)
TA_ATTN_DECODE(ta_attn_decode_kv16_dh64, 64, true)
TA_ATTN_DECODE(ta_attn_decode_kv16_dh128, 128, true)

extern "C" __global__ __launch_bounds__(64) void ta_attn_decode_combine(AttnCombineArgs p) {
  const uint32_t row_id = blockIdx.x, tid = threadIdx.x;
  const uint32_t kvh = row_id / p.group, r = row_id % p.group;
  const uint32_t stride = p.dh + 2;
  const uint64_t row0 = ((uint64_t)kvh * p.num_chunks * p.group + r) * stride;
  const uint64_t step = (uint64_t)p.group * stride;
  float ms = -FLT_MAX;
  for (uint32_t i = 0; i < p.num_chunks; ++i)
    ms = fmaxf(ms, p.scratch[row0 + i * step + p.dh]);
  float l = 0.0f;
  for (uint32_t i = 0; i < p.num_chunks; ++i) {
    const float *c = p.scratch + row0 + i * step;
    l = fmaf(c[p.dh + 1], exp2f(c[p.dh] - ms), l);
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  for (uint32_t d = tid; d < p.dh; d += 64) {
    float num = 0.0f;
    for (uint32_t i = 0; i < p.num_chunks; ++i) {
      const float *c = p.scratch + row0 + i * step;
      num = fmaf(c[d], exp2f(c[p.dh] - ms), num);
    }
    p.out[(uint64_t)row_id * p.dh + d] = num * inv;
  }
}
