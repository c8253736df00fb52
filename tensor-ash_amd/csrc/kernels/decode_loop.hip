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
//  * decode attention, stage 1: workgroup (chunk, kv head) of 4 waves; wave
//    w owns query rows w and w + 4 of the GQA group.  The chunk is walked
//    in 64-position blocks: the four waves stage a block's K^T columns and
//    V rows into LDS with one batch of coalesced loads each (one memory
//    round trip per block; positions past the chunk end are never read and
//    stage as zeros), then every wave computes its rows: lane = position
//    for the scores, lane = head dimension for P @ V.  q (lane = head
//    dimension) and the block's probabilities (lane = position) reach the
//    FMAs through v_readlane as scalar operands.  A wave max per row sets
//    the block's running maximum.  Softmax runs in base 2 (q pre-scaled by
//    scale * log2(e)); the stored max is in log2 units, which stage 2
//    undoes with exp2.
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
  static constexpr int DPL = DH / 64;                 // head dimensions per lane
  static constexpr int RPW = kAttnRows / kAttnWaves;  // query rows per wave
  static constexpr int KPW = DH / kAttnWaves;         // K^T rows each wave stages
  static constexpr int VPW = 64 / kAttnWaves;         // V rows each wave stages
  struct Smem {
    float k[DH][64]; // K^T block: [d][position]
    float v[64][DH]; // V block: [position][d]
  };

  static TA_DEVICE float bcast(float x, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
  }

  static TA_DEVICE void run(const AttnDecodeArgs &p) {
    __shared__ Smem sm;
    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t len = min(p.t_max, p.kv_len + (p.pos ? *p.pos : 0u));
    const uint32_t cs = (len + p.num_chunks - 1) / p.num_chunks;
    const uint32_t p0 = min(chunk * cs, len), p1 = min(p0 + cs, len);
    const uint64_t kt_base = (uint64_t)kvh * DH * p.t_max;
    const uint64_t v_base = (uint64_t)kvh * p.t_max * DH;
    // This wave's rows (wave + 4 i); q pre-scaled by scale * log2(e), lane
    // = head dimension.
    const float scale2 = p.scale * 1.4426950408889634f;
    const bool rows = wave < p.group;
    float qr[RPW][DPL], m[RPW], lp[RPW], acc[RPW][DPL];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const uint32_t r = wave + kAttnWaves * i;
      m[i] = -FLT_MAX;
      lp[i] = 0.0f;
#pragma unroll
      for (int c = 0; c < DPL; ++c) {
        qr[i][c] = r < p.group ? p.q[((uint64_t)kvh * p.group + r) * DH + lane + 64 * c] * scale2 : 0.0f;
        acc[i][c] = 0.0f;
      }
    }

    // Stage one block: wave w loads K^T rows w * KPW .. (lane = position)
    // and V rows w * VPW .. (lane = head dimension), all in one batch.
    // Loads past the chunk end re-read an in-range element and are zeroed
    // when staged, so no load is predicated.  The next block's loads are
    // issued as soon as this one is in LDS, so they run under its compute.
    float kl[KPW], vl[VPW][DPL];
    auto load_block = [&](uint32_t blk) {
      const uint32_t pos = blk + lane;
      const uint32_t kpos = pos < p1 ? pos : blk;
#pragma unroll
      for (int u = 0; u < KPW; ++u)
        kl[u] = load_kv<KV16>(p.kt, kt_base + (uint64_t)(wave * KPW + u) * p.t_max + kpos);
#pragma unroll
      for (int u = 0; u < VPW; ++u) {
        const uint32_t row = min(blk + wave * VPW + u, p1 - 1);
#pragma unroll
        for (int c = 0; c < DPL; ++c)
          vl[u][c] = load_kv<KV16>(p.v, v_base + (uint64_t)row * DH + lane + 64 * c);
      }
    };
    if (p0 < p1)
      load_block(p0);
    for (uint32_t blk = p0; blk < p1; blk += 64) {
      const uint32_t pos = blk + lane;
      const bool valid = pos < p1;
      __syncthreads(); // the previous block's reads are done
#pragma unroll
      for (int u = 0; u < KPW; ++u)
        sm.k[wave * KPW + u][lane] = valid ? kl[u] : 0.0f;
#pragma unroll
      for (int u = 0; u < VPW; ++u)
#pragma unroll
        for (int c = 0; c < DPL; ++c)
          sm.v[wave * VPW + u][lane + 64 * c] = blk + wave * VPW + u < p1 ? vl[u][c] : 0.0f;
      __syncthreads();
      if (blk + 64 < p1)
        load_block(blk + 64);
      if (!rows)
        continue;
      // Scores of this lane's position: q[r][d] from lane d % 64 of its
      // register (v_readlane), K^T from LDS.
      float s[RPW];
#pragma unroll
      for (int i = 0; i < RPW; ++i)
        s[i] = 0.0f;
#pragma unroll
      for (int d = 0; d < DH; ++d) {
        const float k = sm.k[d][lane];
#pragma unroll
        for (int i = 0; i < RPW; ++i)
          s[i] = fmaf(bcast(qr[i][d / 64], d % 64), k, s[i]);
      }
      // Online softmax over the block: one running max per row (uniform
      // over the wave), per-lane partial sums rescaled with it.
      float e[RPW];
#pragma unroll
      for (int i = 0; i < RPW; ++i) {
        const float s2 = valid ? s[i] : -INFINITY;
        const float mn = fmaxf(m[i], wave_max(s2));
        const float corr = exp2f(m[i] - mn);
        e[i] = exp2f(s2 - mn);
        lp[i] = fmaf(lp[i], corr, e[i]);
#pragma unroll
        for (int c = 0; c < DPL; ++c)
          acc[i][c] *= corr;
        m[i] = mn;
      }
      // P @ V: probability j sits in lane j (v_readlane), lane = head
      // dimension for the accumulators.
#pragma unroll
      for (int j = 0; j < 64; ++j) {
        float vv[DPL];
#pragma unroll
        for (int c = 0; c < DPL; ++c)
          vv[c] = sm.v[j][lane + 64 * c];
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
          const float pj = bcast(e[i], j);
#pragma unroll
          for (int c = 0; c < DPL; ++c)
            acc[i][c] = fmaf(pj, vv[c], acc[i][c]);
        }
      }
    }

    // Row state {acc, m, l} to scratch[kv_head][chunk][row].
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const uint32_t r = wave + kAttnWaves * i;
      const float l = wave_sum(lp[i]);
      if (r >= p.group)
        continue;
      float *dst = p.scratch + (((uint64_t)kvh * p.num_chunks + chunk) * p.group + r) * (DH + 2);
#pragma unroll
      for (int c = 0; c < DPL; ++c)
        dst[lane + 64 * c] = acc[i][c];
      if (lane == 0) {
        dst[DH] = m[i];
        dst[DH + 1] = l;
      }
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
  // Quads in batches of 8 per thread, all loads of a batch in flight
  // together (a batch past the end re-reads quad 0 and skips it).
  const uint32_t nq = (reinterpret_cast<uintptr_t>(p.in) & 15u) == 0 ? p.n / 4 : 0;
  constexpr uint32_t QB = 8;
  for (uint32_t q0 = tid; q0 < nq; q0 += QB * kArgmaxThreads) {
    f32x4 v[QB];
#pragma unroll
    for (uint32_t b = 0; b < QB; ++b) {
      const uint32_t q = q0 + b * kArgmaxThreads;
      v[b] = reinterpret_cast<const f32x4 *>(p.in)[q < nq ? q : 0u];
    }
#pragma unroll
    for (uint32_t b = 0; b < QB; ++b) {
      const uint32_t q = q0 + b * kArgmaxThreads;
      if (q < nq) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (v[b][c] >= best) {
            best = v[b][c];
            bi = 4 * q + c;
          }
      }
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
  extern "C" __global__ __launch_bounds__(kAttnThreads)                                \
      __attribute__((amdgpu_waves_per_eu(1, 2))) void NAME(AttnDecodeArgs p) {       \
    AttnDecode<DH, KV16>::run(p);                                                      \
  }
TA_ATTN_DECODE(ta_attn_decode_dh64, 64, false)
TA_ATTN_DECODE(ta_attn_decode_dh128, 128, false)
TA_ATTN_DECODE(ta_attn_decode_kv16_dh64, 64, true)
TA_ATTN_DECODE(ta_attn_decode_kv16_dh128, 128, true)

// One wave per (kv head, row): lane i < num_chunks (<= 32) loads chunk i's
// max and sum, and every lane loads its output columns (d = lane, and
// lane + 64 at head dim 128) of all 32 chunk slots in the same batch
// (slots past num_chunks re-read the last chunk and are not used), so the
// merge costs one memory round trip.  The chunk weights go to LDS; the
// normaliser and each output sum over the chunks in chunk order.
extern "C" __global__ __launch_bounds__(64) void ta_attn_decode_combine(AttnCombineArgs p) {
  constexpr int MAXC = TA_ATTN_DECODE_MAX_CHUNKS;
  static_assert(MAXC <= 64, "one chunk weight per lane of the wave");
  __shared__ float wsh[64], lsh[64];
  const uint32_t row_id = blockIdx.x, lane = threadIdx.x;
  const uint32_t kvh = row_id / p.group, r = row_id % p.group;
  const uint32_t stride = p.dh + 2, nc = p.num_chunks;
  const uint64_t row0 = ((uint64_t)kvh * nc * p.group + r) * stride;
  const uint64_t step = (uint64_t)p.group * stride;
  const bool live = lane < nc;
  const uint32_t lc = live ? lane : 0u;
  float mi = p.scratch[row0 + lc * step + p.dh];
  float li = p.scratch[row0 + lc * step + p.dh + 1];
  const uint32_t d1 = lane + 64u < p.dh ? lane + 64u : lane;
  float o0[MAXC], o1[MAXC];
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const uint64_t at = row0 + (uint64_t)min((uint32_t)i, nc - 1u) * step;
    o0[i] = p.scratch[at + lane];
    o1[i] = p.scratch[at + d1];
  }
  mi = live ? mi : -FLT_MAX;
  li = live ? li : 0.0f;
  const float ms = wave_max(mi);
  wsh[lane] = exp2f(mi - ms);
  lsh[lane] = li;
  __syncthreads();
  float l = 0.0f;
  for (uint32_t i = 0; i < nc; ++i)
    l = fmaf(lsh[i], wsh[i], l);
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  float n0 = 0.0f, n1 = 0.0f;
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    if ((uint32_t)i < nc) {
      n0 = fmaf(o0[i], wsh[i], n0);
      n1 = fmaf(o1[i], wsh[i], n1);
    }
  }
  p.out[(uint64_t)row_id * p.dh + lane] = n0 * inv;
  if (lane + 64u < p.dh)
    p.out[(uint64_t)row_id * p.dh + lane + 64u] = n1 * inv;
}
