// Model ops around the GEMM path for gfx950: row softmax, RMSNorm /
// LayerNorm, RoPE (plain, scattered into a cache, and the prefill QKV
// pack), strided copy and the binary combine (the reference's
// ta_softmax_rows, ta_rms_norm, ta_layer_norm, ta_rope, ta_copy_strided,
// run_rope_scatter, run_prefill_qkv_pack, run_binary;
// src/executor/elementwise/ops.rs with shaders/op_softmax_f32_row.comp,
// op_rmsnorm_body.glsl, op_rope_body.glsl, op_copy_strided_body.glsl).
// All are HBM-bound streaming kernels:
//  * row ops: one 256-thread workgroup per row (grid-strided over rows),
//    128-bit accesses when the row width allows, reductions as a fixed
//    256-wide tree in LDS (the order the reference uses, so results do
//    not depend on scheduling);
//  * RoPE: one thread per rotated pair, f32 rotation with the reference's
//    fma order; partial-rotary lanes copied by the pairs of their vector;
//  * copy: one thread per element, grid-strided, the four f32/f16 pairings.
// exp is the HIP device library's; 1/sqrt is computed as an IEEE divide
// of an IEEE square root.
#include "common.h"

namespace {

constexpr uint32_t kOpThreads = 256;

// Fixed-order tree over the workgroup; every thread gets the result.
template <class F> TA_DEVICE float tree_reduce(float v, float *red, F op) {
  const uint32_t tid = threadIdx.x;
  red[tid] = v;
  __syncthreads();
#pragma unroll
  for (uint32_t stride = kOpThreads / 2; stride > 0; stride >>= 1) {
    if (tid < stride)
      red[tid] = op(red[tid], red[tid + stride]);
    __syncthreads();
  }
  const float r = red[0];
  __syncthreads();
  return r;
}

TA_DEVICE float load_io(const void *p, uint64_t i, bool f16) {
  return f16 ? (float)static_cast<const _Float16 *>(p)[i] : static_cast<const float *>(p)[i];
}
TA_DEVICE void store_io(void *p, uint64_t i, float v, bool f16) {
  if (f16)
    static_cast<_Float16 *>(p)[i] = (_Float16)v;
  else
    static_cast<float *>(p)[i] = v;
}

} // namespace

// Numerically stable softmax with the valid-length mask: max and exp-sum
// passes over the valid columns, then the probabilities (masked columns
// store exactly 0; an all-masked row stores zeros).
extern "C" __global__ __launch_bounds__(kOpThreads) void ta_softmax_rows(SoftmaxArgs p) {
  __shared__ float red[kOpThreads];
  const uint32_t tid = threadIdx.x;
  for (uint32_t row = blockIdx.x; row < p.rows; row += gridDim.x) {
    const uint32_t valid = p.causal ? min(p.cols, p.valid_base + (row % p.rows_per_group) + 1u)
                                    : min(p.cols, p.valid_base);
    const float *in = p.in + (uint64_t)row * p.cols;
    float *out = p.out + (uint64_t)row * p.cols;
    float m = -3.402823466e38f;
    for (uint32_t c = tid; c < valid; c += kOpThreads)
      m = fmaxf(m, in[c] * p.scale);
    const float row_max = tree_reduce(m, red, [](float a, float b) { return fmaxf(a, b); });
    float s = 0.0f;
    for (uint32_t c = tid; c < valid; c += kOpThreads)
      s += expf(in[c] * p.scale - row_max);
    const float sum = tree_reduce(s, red, [](float a, float b) { return a + b; });
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (uint32_t c = tid; c < p.cols; c += kOpThreads)
      out[c] = c < valid ? expf(in[c] * p.scale - row_max) * inv : 0.0f;
  }
}

// RMSNorm (bias null): out = x * r * w; LayerNorm: out = (x - mean) * r * w
// + b; r = 1 / sqrt(mean((x - mean)^2) + eps) with mean = 0 for RMSNorm.
// In-place safe: each element is read before the thread writes it and no
// thread reads another's column after the reductions.
extern "C" __global__ __launch_bounds__(kOpThreads) void ta_norm_rows(NormArgs p) {
  __shared__ float red[kOpThreads];
  const uint32_t tid = threadIdx.x;
  const bool f16 = p.io_f16 != 0;
  const bool layer = p.bias != nullptr;
  const bool vec = !f16 && (p.cols & 3u) == 0u;
  const float inv_n = 1.0f / (float)p.cols;
  for (uint32_t row = blockIdx.x; row < p.rows; row += gridDim.x) {
    const uint64_t base = (uint64_t)row * p.cols;
    float mean = 0.0f;
    if (layer) {
      float local = 0.0f;
      if (vec) {
        const f32x4 *in4 = reinterpret_cast<const f32x4 *>(static_cast<const float *>(p.in) + base);
        for (uint32_t c = tid; c < p.cols / 4; c += kOpThreads) {
          const f32x4 v = in4[c];
          local += ((v[0] + v[1]) + v[2]) + v[3];
        }
      } else {
        for (uint32_t c = tid; c < p.cols; c += kOpThreads)
          local += load_io(p.in, base + c, f16);
      }
      mean = tree_reduce(local, red, [](float a, float b) { return a + b; }) * inv_n;
    }
    float sq = 0.0f;
    if (vec) {
      const f32x4 *in4 = reinterpret_cast<const f32x4 *>(static_cast<const float *>(p.in) + base);
      for (uint32_t c = tid; c < p.cols / 4; c += kOpThreads) {
        const f32x4 v = in4[c];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float d = v[e] - mean;
          sq = fmaf(d, d, sq);
        }
      }
    } else {
      for (uint32_t c = tid; c < p.cols; c += kOpThreads) {
        const float d = load_io(p.in, base + c, f16) - mean;
        sq = fmaf(d, d, sq);
      }
    }
    const float r =
        1.0f / sqrtf(tree_reduce(sq, red, [](float a, float b) { return a + b; }) * inv_n + p.eps);
    if (vec) {
      const f32x4 *in4 = reinterpret_cast<const f32x4 *>(static_cast<const float *>(p.in) + base);
      f32x4 *out4 = reinterpret_cast<f32x4 *>(static_cast<float *>(p.out) + base);
      const f32x4 *w4 = reinterpret_cast<const f32x4 *>(p.weight);
      const f32x4 *b4 = reinterpret_cast<const f32x4 *>(p.bias);
      for (uint32_t c = tid; c < p.cols / 4; c += kOpThreads) {
        const f32x4 x = in4[c], w = w4[c];
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = (x[e] - mean) * r * w[e];
        if (layer) {
          const f32x4 b = b4[c];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            v[e] += b[e];
        }
        out4[c] = v;
      }
    } else {
      for (uint32_t c = tid; c < p.cols; c += kOpThreads) {
        float v = (load_io(p.in, base + c, f16) - mean) * r * p.weight[c];
        if (layer)
          v += p.bias[c];
        store_io(p.out, base + c, v, f16);
      }
    }
  }
}

// One thread per rotated pair (grid-strided): r0 = fma(x0, c, -x1 s),
// r1 = fma(x0, s, x1 c); lanes past rot_dim are copied by the pairs of
// their head vector.  A device position past the table skips the pair.  Each element is read and written by one thread, so
// in-place is safe.
// One thread per rotated pair of a [tokens, heads, head_dim] input:
// put(token, head, dim, value) receives the pair's two rotated values (the
// reference's fma order) and the pass-through lanes the pair owns.
template <class Put> TA_DEVICE void rope_pairs(const RopeArgs &p, bool f16, Put &&put) {
  const uint32_t half = p.rot_dim / 2;
  const uint64_t pairs = (uint64_t)p.tokens * p.heads * half;
  const uint32_t pos0 = p.pos_base + (p.pos_addr ? *p.pos_addr : 0u);
  for (uint64_t id = (uint64_t)blockIdx.x * kOpThreads + threadIdx.x; id < pairs;
       id += (uint64_t)gridDim.x * kOpThreads) {
    const uint32_t pair = (uint32_t)(id % half);
    const uint64_t vecid = id / half; // token * heads + head
    const uint32_t token = (uint32_t)(vecid / p.heads), head = (uint32_t)(vecid % p.heads);
    const uint64_t vbase = vecid * p.head_dim;
    const uint64_t i0 = vbase + 2 * pair;
    const float x0 = load_io(p.in, i0, f16), x1 = load_io(p.in, i0 + 1, f16);
    const uint64_t angle = ((uint64_t)(pos0 + token) * half + pair) * 2;
    if (angle + 1 >= p.table_len)
      continue;
    const float c = p.table[angle], s = p.table[angle + 1];
    put(token, head, 2 * pair, fmaf(x0, c, -x1 * s));
    put(token, head, 2 * pair + 1, fmaf(x0, s, x1 * c));
    for (uint32_t lane = pair; lane < p.head_dim - p.rot_dim; lane += half)
      put(token, head, p.rot_dim + lane, load_io(p.in, vbase + p.rot_dim + lane, f16));
  }
}

extern "C" __global__ __launch_bounds__(kOpThreads) void ta_rope(RopeArgs p) {
  const bool f16 = p.io_f16 != 0;
  rope_pairs(p, f16, [&](uint32_t token, uint32_t head, uint32_t dim, float v) {
    store_io(p.out, ((uint64_t)token * p.heads + head) * p.head_dim + dim, v, f16);
  });
}

// src/executor/elementwise/ops.rs:243-316 (run_rope_scatter): the RoPE
// above with each element stored at its strided cache location.
extern "C" __global__ __launch_bounds__(kOpThreads) void ta_rope_scatter(RopeScatterArgs p) {
  const uint64_t base =
      p.dst_offset + (uint64_t)(p.rope.pos_addr ? *p.rope.pos_addr : 0u) * p.pos_scale;
  rope_pairs(p.rope, false, [&](uint32_t token, uint32_t head, uint32_t dim, float v) {
    const uint64_t d = base + (uint64_t)token * p.dst_strides[0] +
                       (uint64_t)head * p.dst_strides[1] + (uint64_t)dim * p.dst_strides[2];
    if (d < p.dst_len)
      store_io(p.dst, d, v, p.dst_f16 != 0);
  });
}

// src/executor/elementwise/ops.rs:318-380 (run_binary): four elements per
// thread, grid-strided; SiLU with the library exp and an IEEE divide.
extern "C" __global__ __launch_bounds__(kOpThreads) void ta_binary(BinaryArgs p) {
  const bool f16 = p.io_f16 != 0;
  for (uint64_t i = ((uint64_t)blockIdx.x * kOpThreads + threadIdx.x) * 4; i < p.n;
       i += (uint64_t)gridDim.x * kOpThreads * 4) {
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) {
      if (i + c >= p.n)
        break;
      const float a = load_io(p.a, i + c, f16), b = load_io(p.b, i + c, f16);
      const float v = p.mode == 0 ? fmaf(p.beta, b, a) : (a / (1.0f + expf(-a))) * b;
      store_io(p.out, i + c, v, f16);
    }
  }
}

// src/executor/elementwise/flash.rs:255-402 (run_prefill_qkv_pack): the
// work is Q pairs, then K pairs, then V quads, one item per thread
// (grid-strided); rotations as ta_rope (f32 math, RNE store).
extern "C" __global__ __launch_bounds__(kOpThreads) void ta_prefill_qkv_pack(QkvPackArgs args) {
  struct {
    const _Float16 *qkv;
    _Float16 *q, *kt, *v;
  } h{reinterpret_cast<const _Float16 *>(args.qkv), reinterpret_cast<_Float16 *>(args.q),
      reinterpret_cast<_Float16 *>(args.kt), reinterpret_cast<_Float16 *>(args.v)};
  const QkvPackArgs &p = args;
  const uint32_t half = p.rot_dim / 2, tail = p.head_dim - p.rot_dim;
  const uint64_t q_pairs = (uint64_t)p.tokens * p.heads * half;
  const uint64_t k_pairs = (uint64_t)p.tokens * p.kv_heads * half;
  const uint64_t v_quads = (uint64_t)p.tokens * p.kv_heads * (p.head_dim / 4);
  const uint64_t total = q_pairs + k_pairs + v_quads;
  for (uint64_t id = (uint64_t)blockIdx.x * kOpThreads + threadIdx.x; id < total;
       id += (uint64_t)gridDim.x * kOpThreads) {
    if (id < q_pairs + k_pairs) {
      const bool is_q = id < q_pairs;
      const uint64_t kid = is_q ? id : id - q_pairs;
      const uint32_t nh = is_q ? p.heads : p.kv_heads;
      const uint32_t pair = (uint32_t)(kid % half);
      const uint32_t head = (uint32_t)((kid / half) % nh);
      const uint32_t token = (uint32_t)(kid / ((uint64_t)half * nh));
      const uint64_t src = (uint64_t)token * p.qkv_stride + (is_q ? 0u : p.k_offset) +
                           (uint64_t)head * p.head_dim;
      const float x0 = (float)h.qkv[src + 2 * pair], x1 = (float)h.qkv[src + 2 * pair + 1];
      const uint64_t angle = ((uint64_t)(p.pos_base + token) * half + pair) * 2;
      const float c = p.table[angle], s = p.table[angle + 1];
      const _Float16 y0 = (_Float16)fmaf(x0, c, -x1 * s), y1 = (_Float16)fmaf(x0, s, x1 * c);
      const uint32_t pos = p.pos_base + token;
      if (is_q) {
        const uint64_t dst = ((uint64_t)head * p.tokens + token) * p.head_dim;
        h.q[dst + 2 * pair] = y0;
        h.q[dst + 2 * pair + 1] = y1;
        for (uint32_t lane = pair; lane < tail; lane += half)
          h.q[dst + p.rot_dim + lane] = h.qkv[src + p.rot_dim + lane];
      } else {
        const uint64_t col = (uint64_t)head * p.head_dim;
        h.kt[(col + 2 * pair) * p.t_max + pos] = y0;
        h.kt[(col + 2 * pair + 1) * p.t_max + pos] = y1;
        for (uint32_t lane = pair; lane < tail; lane += half)
          h.kt[(col + p.rot_dim + lane) * p.t_max + pos] = h.qkv[src + p.rot_dim + lane];
      }
    } else {
      const uint64_t vid = id - q_pairs - k_pairs;
      const uint32_t n4 = p.head_dim / 4;
      const uint32_t d4 = (uint32_t)(vid % n4);
      const uint32_t head = (uint32_t)((vid / n4) % p.kv_heads);
      const uint32_t token = (uint32_t)(vid / ((uint64_t)n4 * p.kv_heads));
      const uint64_t src = (uint64_t)token * p.qkv_stride + p.v_offset + (uint64_t)head * p.head_dim;
      const uint64_t dst = ((uint64_t)head * p.t_max + p.pos_base + token) * p.head_dim;
      *reinterpret_cast<f16x4 *>(h.v + dst + 4 * d4) =
          *reinterpret_cast<const f16x4 *>(h.qkv + src + 4 * d4);
    }
  }
}

extern "C" __global__ __launch_bounds__(kOpThreads) void ta_copy_strided(CopyArgs p) {
  const uint64_t plane = (uint64_t)p.extent[0] * p.extent[1];
  const uint64_t total = plane * p.extent[2];
  const uint64_t shift = (uint64_t)(p.pos_addr ? *p.pos_addr : 0u) * p.pos_scale;
  for (uint64_t id = (uint64_t)blockIdx.x * kOpThreads + threadIdx.x; id < total;
       id += (uint64_t)gridDim.x * kOpThreads) {
    const uint64_t x = id % p.extent[0], y = (id / p.extent[0]) % p.extent[1], z = id / plane;
    const uint64_t s = p.src_offset + x * p.src_strides[0] + y * p.src_strides[1] +
                       z * p.src_strides[2];
    const uint64_t d = p.dst_offset + shift + x * p.dst_strides[0] + y * p.dst_strides[1] +
                       z * p.dst_strides[2];
    if (d < p.dst_len)
      store_io(p.dst, d, load_io(p.src, s, p.src_f16 != 0), p.dst_f16 != 0);
  }
}
