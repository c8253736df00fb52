// Fused causal prefill attention for gfx950 (the reference's
// run_flash_attention: src/executor/elementwise/flash.rs:13-250,
// shaders/attention_flash_kernel.glsl).  out = softmax_causal(q K^T *
// scale) V in one launch with an online softmax; score tiles stay in
// registers and tiles past a workgroup's causal frontier are never read.
//
// Work split.  A workgroup is QB*KP waves over 32*QB query rows of one
// head: wave w takes query block w % QB (32 rows) and key part w / QB (32
// keys) of every 32*KP-key tile, keeping its own running max / sum /
// output; the KP key parts of a query block merge through LDS at the end,
// in part order.  QB = 2 (64-row tiles).  Head dim 64: KP = 4 (8 waves;
// each wave's walk over the keys is half as long as with 2 parts: 10%
// faster on a 512-token prompt; 32-row tiles with 4 parts, twice the
// workgroups, were 10-20% slower).  Head dim 128: KP = 2 (a 128-key f32
// K/V tile would take 128 KiB of LDS).
//
// Operands (all v_mfma_f32_32x32x2_f32, f32 in f32 accumulate, so f16
// caches widen exactly and the result is f32-accurate):
//  * scores are computed transposed, S^T = K Q^T (m = key, n = query,
//    k = head dim): each lane then owns one query row, so the row max is
//    a register reduction plus one exchange between the lane halves.
//    MFMA step s pairs head-dim lanes s and s + dh/2 (lane half h takes
//    d = s + h*dh/2), so every lane keeps its query row's q values for
//    its half of the head dim in registers;
//  * O^T += V^T P^T (m = head dim, n = query, k = key): in the score
//    accumulator lane (j, h) holds keys 8q + 4h + r at register 4q + r,
//    so step (q, r), which pairs keys 8q + r and 8q + 4 + r, takes its
//    P operand straight from register 4q + r in both lane halves; no
//    data moves between the two products.
// K and V tiles are staged in LDS as [d][key] and [key][d] (the cache
// layouts), so each MFMA operand read is 32 consecutive floats per lane
// half.  Cache rows at or past min(t_max, the workgroup's frontier) are
// staged as zeros, so unwritten cache memory never reaches the sums.
#include "common.h"

#include <type_traits>

namespace {

template <int DH> constexpr int flash_parts() { return ta_flash_parts(DH); }     // KP
template <int DH> constexpr int flash_qblocks() { return ta_flash_qblocks(DH); } // QB
constexpr float kNegMax = -3.402823466e38f;

template <bool F16> TA_DEVICE f32x4 load4(const void *base, uint64_t i) {
  if constexpr (F16) {
    const f16x4 h = *reinterpret_cast<const f16x4 *>(static_cast<const _Float16 *>(base) + i);
    return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
  } else {
    return *reinterpret_cast<const f32x4 *>(static_cast<const float *>(base) + i);
  }
}
// Cache loads in storage type; widened to f32 only when written to LDS,
// so a prefetch does not wait for its data at the load.
template <bool F16> TA_DEVICE auto load_raw(const void *base, uint64_t i) {
  if constexpr (F16)
    return *reinterpret_cast<const f16x4 *>(static_cast<const _Float16 *>(base) + i);
  else
    return *reinterpret_cast<const f32x4 *>(static_cast<const float *>(base) + i);
}
template <bool F16> TA_DEVICE auto load_raw1(const void *base, uint64_t i) {
  if constexpr (F16)
    return static_cast<const _Float16 *>(base)[i];
  else
    return static_cast<const float *>(base)[i];
}
TA_DEVICE f32x4 widen(f32x4 v) { return v; }
TA_DEVICE f32x4 widen(f16x4 h) { return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]}; }

template <bool F16> TA_DEVICE void store4(void *base, uint64_t i, f32x4 v) {
  if constexpr (F16) {
    *reinterpret_cast<f16x4 *>(static_cast<_Float16 *>(base) + i) =
        f16x4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
  } else {
    *reinterpret_cast<f32x4 *>(static_cast<float *>(base) + i) = v;
  }
}

template <int DH, bool KV16, bool IO16> TA_DEVICE void flash_body(const FlashArgs &p) {
  constexpr int KP = flash_parts<DH>();  // key parts
  constexpr int QB = flash_qblocks<DH>(); // 32-row query blocks
  constexpr int kBQ = 32 * QB;           // query rows per workgroup
  constexpr int kFlashThreads = 64 * QB * KP;
  constexpr int kBK = 32 * KP;           // keys per tile
  constexpr int KC = kBK / 4;            // four-key chunks per K row
  constexpr int HALF = DH / 2; // MFMA k-steps of the score product
  constexpr int DB = DH / 32;  // 32-row head-dim blocks of the output
  constexpr int REGS = DB * 16 + 2; // merge record per lane: o, m, l
  constexpr int LDS_TILES = 2 * DH * kBK, LDS_MERGE = QB * (KP - 1) * REGS * 64;
  __shared__ float lds[LDS_TILES > LDS_MERGE ? LDS_TILES : LDS_MERGE];
  float *ksh = lds;            // [DH][kBK]
  float *vsh = lds + DH * kBK; // [kBK][DH]

  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t qb = wave % QB, kh = wave / QB;
  const uint32_t j = lane & 31u, h = lane >> 5;

  // Workgroups of one head run on one XCD (its L2 keeps that head's K/V);
  // within a head the longest (latest) query tiles start first.
  const uint32_t total = p.q_tiles * p.heads;
  uint32_t pidx = blockIdx.x;
  if (total % 8u == 0u)
    pidx = (blockIdx.x & 7u) * (total >> 3) + (blockIdx.x >> 3);
  const uint32_t head = pidx / p.q_tiles;
  const uint32_t tile = p.q_tiles - 1u - pidx % p.q_tiles;

  const uint32_t q0 = tile * kBQ;
  const uint32_t qrow = q0 + qb * 32u + j;
  const bool live = qrow < p.t_q;
  const uint32_t kv_head = head / p.group_size;
  const uint32_t valid_row = live ? min(p.kv_len, p.pos_base + qrow + 1u) : 0u;
  const uint32_t last_row = min(q0 + (uint32_t)kBQ, p.t_q) - 1u;
  const uint32_t valid_max = min(p.kv_len, p.pos_base + last_row + 1u);
  const uint32_t stage_end = min(valid_max, p.t_max);
  const uint32_t n_tiles = (valid_max + kBK - 1u) / kBK;

  // This lane's q values: Q[qrow][h*HALF + s], s < HALF.
  float qreg[HALF];
  {
    const uint64_t qbase = (uint64_t)head * p.q_head_stride +
                           (uint64_t)min(qrow, p.t_q - 1u) * p.q_row_stride + h * HALF;
#pragma unroll
    for (int s = 0; s < HALF; s += 4) {
      const f32x4 v = load4<IO16>(p.q, qbase + s);
      qreg[s] = v[0];
      qreg[s + 1] = v[1];
      qreg[s + 2] = v[2];
      qreg[s + 3] = v[3];
    }
  }

  f32x16 o[DB];
#pragma unroll
  for (int b = 0; b < DB; ++b)
    o[b] = f32x16{};
  float m_run = kNegMax, l_run = 0.0f;

  const uint64_t kt_base = (uint64_t)kv_head * DH * p.t_max;
  const uint64_t v_base = (uint64_t)kv_head * p.t_max * DH;
  const bool kt_vec = (p.t_max & 3u) == 0u;

  // K/V of the next tile are loaded into registers while the current one
  // is computed: ksh[d][c] = Kt[d][k0 + c] in KC four-key chunks per row,
  // vsh[r][d] = V[k0 + r][d].
  constexpr int NCH = DH * kBK / 4 / kFlashThreads;
  using Raw = typename std::conditional<KV16, f16x4, f32x4>::type; // widened at the LDS store
  Raw kreg[NCH], vreg[NCH];
  auto load_tile = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const uint32_t c = tid + i * kFlashThreads;
      const uint32_t d = c / KC, key = k0 + (c % KC) * 4u;
      const uint64_t src = kt_base + (uint64_t)d * p.t_max + key;
      if (kt_vec && key + 3u < stage_end) {
        kreg[i] = load_raw<KV16>(p.kt, src);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          kreg[i][e] = key + e < stage_end ? load_raw1<KV16>(p.kt, src + e) : 0;
      }
    }
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const uint32_t c = tid + i * kFlashThreads;
      const uint32_t key = k0 + c / (DH / 4), dc = (c % (DH / 4)) * 4u;
      vreg[i] = key < stage_end ? load_raw<KV16>(p.v, v_base + (uint64_t)key * DH + dc) : Raw{};
    }
  };
  if (n_tiles > 0)
    load_tile(0);

  // Softmax in base 2: scores are scaled by scale * log2(e) once, so each
  // probability is one native exp2.
  const float scale2 = p.scale * 1.44269504088896340736f;

  for (uint32_t t = 0; t < n_tiles; ++t) {
    const uint32_t k0 = t * kBK;
    __syncthreads(); // the previous tile's LDS reads are done
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const uint32_t c = tid + i * kFlashThreads;
      *reinterpret_cast<f32x4 *>(ksh + (c / KC) * kBK + (c % KC) * 4u) = widen(kreg[i]);
      *reinterpret_cast<f32x4 *>(vsh + (c / (DH / 4)) * DH + (c % (DH / 4)) * 4u) = widen(vreg[i]);
    }
    __syncthreads();
    if (t + 1 < n_tiles)
      load_tile(k0 + kBK);

    // S^T block: keys kh*32 + m (m < 32) against this wave's 32 queries.
    f32x16 s = f32x16{};
    {
      const float *kp = ksh + h * HALF * kBK + kh * 32u + j;
#pragma unroll
      for (int st = 0; st < HALF; ++st)
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kp[st * kBK], qreg[st], s, 0, 0, 0);
    }

    // Online softmax over this wave's keys (per query row = per lane pair).
    const uint32_t kbase = k0 + kh * 32u + 4u * h;
    float tmax = kNegMax;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t key = kbase + 8u * q + r;
        const float v = key < valid_row ? s[4 * q + r] * scale2 : kNegMax;
        s[4 * q + r] = v;
        tmax = fmaxf(tmax, v);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    const float corr = exp2f(m_run - m_new);
    float psum = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t key = kbase + 8u * q + r;
        const float pv = key < valid_row ? exp2f(s[4 * q + r] - m_new) : 0.0f;
        s[4 * q + r] = pv;
        psum += pv;
      }
    l_run = l_run * corr + psum;
    m_run = m_new;
#pragma unroll
    for (int b = 0; b < DB; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        o[b][e] *= corr;

    // O^T += V^T P^T over this wave's 32 keys.
    {
      const float *vp = vsh + (kh * 32u + 4u * h) * DH + j;
#pragma unroll
      for (int b = 0; b < DB; ++b)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vp[(8 * q + r) * DH + b * 32], s[4 * q + r],
                                                        o[b], 0, 0, 0);
    }
  }

  // Merge the key parts of each query block: parts 1..KP-1 leave their
  // state as [register][lane] records in LDS, part 0 rescales all KP to
  // the common maximum and sums them in part order.
  __syncthreads();
  float *mb = lds + qb * ((KP - 1) * REGS * 64);
  if (kh != 0u) {
    float *rec = mb + (kh - 1u) * (REGS * 64);
#pragma unroll
    for (int b = 0; b < DB; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        rec[(b * 16 + e) * 64 + lane] = o[b][e];
    rec[(DB * 16) * 64 + lane] = m_run;
    rec[(DB * 16 + 1) * 64 + lane] = l_run;
  }
  __syncthreads();
  if (kh == 0u) {
    float mp[KP], a[KP];
    mp[0] = m_run;
    float m = m_run;
#pragma unroll
    for (int k = 1; k < KP; ++k) {
      mp[k] = mb[((k - 1) * REGS + DB * 16) * 64 + lane];
      m = fmaxf(m, mp[k]);
    }
    float l = 0.0f;
#pragma unroll
    for (int k = 0; k < KP; ++k) {
      a[k] = exp2f(mp[k] - m);
      const float lk = k == 0 ? l_run : mb[((k - 1) * REGS + DB * 16 + 1) * 64 + lane];
      l = k == 0 ? lk * a[k] : l + lk * a[k];
    }
    l += __shfl_xor(l, 32);
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    if (live) {
      const uint64_t obase =
          (uint64_t)head * p.o_head_stride + (uint64_t)qrow * p.o_row_stride + 4u * h;
#pragma unroll
      for (int b = 0; b < DB; ++b)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          f32x4 v;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int e = b * 16 + 4 * q + r;
            float acc = o[b][4 * q + r] * a[0];
#pragma unroll
            for (int k = 1; k < KP; ++k)
              acc += mb[((k - 1) * REGS + e) * 64 + lane] * a[k];
            v[r] = acc * inv;
          }
          store4<IO16>(p.out, obase + b * 32 + 8 * q, v);
        }
    }
  }
}

} // namespace

#define TA_FLASH(NAME, DH, KV16, IO16)                                                     \
  extern "C" __global__ __launch_bounds__(64 * flash_qblocks<DH>() * flash_parts<DH>()) void NAME(FlashArgs p) { \
    flash_body<DH, KV16, IO16>(p);                                                         \
  }

TA_FLASH(ta_flash_attention_dh64, 64, false, false)
TA_FLASH(ta_flash_attention_dh128, 128, false, false)
TA_FLASH(ta_flash_attention_kv16_dh64, 64, true, false)
TA_FLASH(ta_flash_attention_kv16_dh128, 128, true, false)
TA_FLASH(ta_flash_attention_io16_dh64, 64, true, true)
TA_FLASH(ta_flash_attention_io16_dh128, 128, true, true)
