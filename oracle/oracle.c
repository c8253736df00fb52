/*
 * CPU oracle for the fused-epilogue GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links or calls
 * this file; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load liboracle.so, and only as the checker (or as the
 * timed CPU baseline), never as the thing measured or shipped.
 *
 * Each function restates one piece of the reference's CPU-side algorithm
 * (gusahlg/tensor-ash) in plain C and cites the file:line it follows.  The
 * reference is Rust and cannot be compiled in this image (no cargo/rustc),
 * so there is no oracle/_ref build; how each function is pinned is listed
 * in the pinning table of tests/test_oracle.py:
 *
 *   fill_det / LcgRng        properties from tools/test-support/src/lib.rs
 *                            :168-193 + moments; exact stream has no golden
 *                            values in the reference  -> "parity unpinned"
 *                            for the exact bit stream (inputs only; GPU
 *                            parity never depends on it)
 *   cpu_bmm                  reference KATs (lib.rs:221-277) + numpy f64
 *   max_abs_err, tolerance   reference KATs (lib.rs:205-218,280-291)
 *   f16 encode/decode        reference KATs (src/dtype.rs:118-163) + numpy
 *                            float16 (IEEE RNE) bit-exact over 2^20 samples
 *   pack_f16w_row_tiles      reference KAT (src/matmul/api.rs:355-380)
 *   epilogue                 closed forms (ReLU, sigmoid identity, torch
 *                            gelu(approximate="tanh")) + c_smoke KAT
 *   split-K partition        invariants (exact cover, sizes differ <= 1)
 *   fill_normal              own definition (Box-Muller over the LCG);
 *                            pinned by moments / KS test only
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define LCG_MUL 6364136223846793005ULL
#define LCG_ADD 1442695040888963407ULL
#define SEED_MIX 0x9E3779B97F4A7C15ULL

/* tools/test-support/src/lib.rs:9-18: 64-bit LCG, top 24 bits of state
 * after each step mapped to [-1, 1). */
void ta_oracle_fill_det(float *out, size_t len, uint64_t seed) {
  uint64_t s = (seed * SEED_MIX) | 1ULL;
  for (size_t i = 0; i < len; ++i) {
    s = s * LCG_MUL + LCG_ADD;
    uint32_t bits = (uint32_t)(s >> 40);
    out[i] = (float)bits / (float)(1u << 24) * 2.0f - 1.0f;
  }
}

/* tools/test-support/src/lib.rs:26-55 (LcgRng::new / next_u64 /
 * range_u32): writes `count` draws of range_u32(lo, hi). */
int ta_oracle_lcg_range(uint64_t seed, uint32_t lo, uint32_t hi, uint32_t *out,
                        size_t count) {
  if (lo > hi)
    return -1;
  uint64_t state = (seed * SEED_MIX) | 1ULL;
  for (size_t i = 0; i < count; ++i) {
    if (lo == hi) {
      out[i] = lo;
      continue;
    }
    state = state * LCG_MUL + LCG_ADD;
    uint64_t span = (uint64_t)(hi - lo) + 1ULL;
    out[i] = lo + (uint32_t)(state % span);
  }
  return 0;
}

/* Gaussian inputs for the benchmark configs.  The reference has no
 * Gaussian generator; this is this project's own definition: the same LCG
 * as fill_det, two 24-bit uniforms per pair, Box-Muller in double,
 * scaled by `stddev`.  u1 = (b1 + 1) / 2^24 lies in (0, 1] so log(u1) is
 * finite. */
void ta_oracle_fill_normal(float *out, size_t len, uint64_t seed,
                           float stddev) {
  uint64_t s = (seed * SEED_MIX) | 1ULL;
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = 0; i < len; i += 2) {
    s = s * LCG_MUL + LCG_ADD;
    double u1 = ((double)(uint32_t)(s >> 40) + 1.0) / 16777216.0;
    s = s * LCG_MUL + LCG_ADD;
    double u2 = (double)(uint32_t)(s >> 40) / 16777216.0;
    double r = sqrt(-2.0 * log(u1));
    out[i] = (float)(r * cos(two_pi * u2) * (double)stddev);
    if (i + 1 < len)
      out[i + 1] = (float)(r * sin(two_pi * u2) * (double)stddev);
  }
}

/* One output row of tools/test-support/src/lib.rs:66-135 (cpu_bmm): f64
 * accumulation over k in ascending order, cast to f32, times alpha in f32,
 * plus the old C value in f32 when accumulating.  The loops run k-outer /
 * j-inner over a row of f64 accumulators so B is read contiguously; every
 * output still adds its K products in the same (ascending k) order as the
 * reference's j-outer / k-inner loop, so the result is bit-identical. */
static void bmm_row(const float *a, const float *b, float *c, uint32_t n,
                    uint32_t k, float alpha, int accumulate, double *acc) {
  for (uint32_t j = 0; j < n; ++j)
    acc[j] = 0.0;
  for (uint32_t kk = 0; kk < k; ++kk) {
    const double av = (double)a[kk];
    const float *brow = b + (size_t)kk * n;
    for (uint32_t j = 0; j < n; ++j)
      acc[j] += av * (double)brow[j];
  }
  for (uint32_t j = 0; j < n; ++j) {
    float scaled = alpha * (float)acc[j];
    c[j] = accumulate ? c[j] + scaled : scaled;
  }
}

/* The reference's own loop order (j outer, k inner; lib.rs:113-127), kept
 * for timing the CPU baseline; same sums in the same order as bmm_row. */
static void bmm_row_ijk(const float *a, const float *b, float *c, uint32_t n,
                        uint32_t k, float alpha) {
  for (uint32_t j = 0; j < n; ++j) {
    double acc = 0.0;
    for (uint32_t kk = 0; kk < k; ++kk)
      acc += (double)a[kk] * (double)b[(size_t)kk * n + j];
    c[j] = alpha * (float)acc;
  }
}

static int bmm_check(size_t a_len, size_t b_len, uint32_t batch, uint32_t m,
                     uint32_t n, uint32_t k, int *a_batched,
                     int *b_batched) {
  size_t mk = (size_t)m * k, kn = (size_t)k * n;
  *a_batched = a_len == (size_t)batch * mk;
  *b_batched = b_len == (size_t)batch * kn;
  if (!*a_batched && a_len != mk)
    return -1;
  if (!*b_batched && b_len != kn)
    return -2;
  return 0;
}

/* tools/test-support/src/lib.rs:66-135.  `out` holds batch*m*n floats; when
 * `c_init` is non-null it is copied to `out` first.  An input whose length
 * is one plane is broadcast over the batch.  Returns 0, or <0 on a shape
 * mismatch (the reference panics). */
int ta_oracle_cpu_bmm(const float *a, size_t a_len, const float *b,
                      size_t b_len, const float *c_init, uint32_t batch,
                      uint32_t m, uint32_t n, uint32_t k, float alpha,
                      int accumulate, float *out) {
  int ab, bb;
  int rc = bmm_check(a_len, b_len, batch, m, n, k, &ab, &bb);
  if (rc)
    return rc;
  size_t mk = (size_t)m * k, kn = (size_t)k * n, mn = (size_t)m * n;
  if (c_init)
    memmove(out, c_init, (size_t)batch * mn * sizeof(float));
  else
    memset(out, 0, (size_t)batch * mn * sizeof(float));
  double *acc = (double *)malloc((size_t)n * sizeof(double));
  if (!acc)
    return -3;
  for (uint32_t bi = 0; bi < batch; ++bi)
    for (uint32_t i = 0; i < m; ++i)
      bmm_row(a + (ab ? bi * mk : 0) + (size_t)i * k, b + (bb ? bi * kn : 0),
              out + bi * mn + (size_t)i * n, n, k, alpha, accumulate, acc);
  free(acc);
  return 0;
}

/* The same computation parallelised over (batch, row) with OpenMP.  Rows
 * are independent and each row runs the serial inner loops, so the output
 * is bit-identical to ta_oracle_cpu_bmm.  Used as the multi-core CPU
 * baseline.  `row_begin`/`row_end` bound the flattened (batch*m) row range
 * that is computed (the rest of `out` is left untouched), so a bounded
 * sample of a large GEMM can be timed.  ijk != 0 runs the reference's own
 * j-outer / k-inner loop order (the timed CPU baseline); 0 runs the
 * cache-friendly order with identical results. */
int ta_oracle_cpu_bmm_rows(const float *a, size_t a_len, const float *b,
                           size_t b_len, uint32_t batch, uint32_t m,
                           uint32_t n, uint32_t k, float alpha, float *out,
                           uint64_t row_begin, uint64_t row_end,
                           int threads, int ijk) {
  int ab, bb;
  int rc = bmm_check(a_len, b_len, batch, m, n, k, &ab, &bb);
  if (rc)
    return rc;
  size_t mk = (size_t)m * k, kn = (size_t)k * n, mn = (size_t)m * n;
  uint64_t total = (uint64_t)batch * m;
  if (row_end > total)
    row_end = total;
#ifdef _OPENMP
  if (threads > 0)
    omp_set_num_threads(threads);
#endif
  int failed = 0;
#ifdef _OPENMP
#pragma omp parallel reduction(| : failed)
#endif
  {
    double *acc = (double *)malloc((size_t)n * sizeof(double));
    if (!acc) {
      failed = 1;
    } else {
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
      for (int64_t r = (int64_t)row_begin; r < (int64_t)row_end; ++r) {
        uint64_t bi = (uint64_t)r / m, i = (uint64_t)r % m;
        if (ijk)
          bmm_row_ijk(a + (ab ? bi * mk : 0) + i * k, b + (bb ? bi * kn : 0),
                      out + bi * mn + i * n, n, k, alpha);
        else
          bmm_row(a + (ab ? bi * mk : 0) + i * k, b + (bb ? bi * kn : 0),
                  out + bi * mn + i * n, n, k, alpha, 0, acc);
      }
      free(acc);
    }
  }
  (void)threads;
  return failed ? -3 : 0;
}

int ta_oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* tools/test-support/src/lib.rs:140-155.  Positional max |a-b|; a
 * non-finite difference reports +inf at its index. */
float ta_oracle_max_abs_err(const float *a, const float *b, size_t len,
                            size_t *index) {
  float best = 0.0f;
  size_t idx = 0;
  for (size_t i = 0; i < len; ++i) {
    float e = fabsf(a[i] - b[i]);
    if (!isfinite(e)) {
      if (index)
        *index = i;
      return INFINITY;
    }
    if (e > best) {
      best = e;
      idx = i;
    }
  }
  if (index)
    *index = idx;
  return best;
}

/* tools/test-support/src/lib.rs:160-162: 8 * K * f32::EPSILON. */
float ta_oracle_tolerance(uint32_t k) {
  return 8.0f * (float)k * 1.1920928955078125e-7f;
}

/* src/dtype.rs:42-84: f32 -> binary16, round to nearest even; overflow to
 * signed inf; NaN keeps a quiet-NaN payload bit. */
uint16_t ta_oracle_f32_to_f16(float value) {
  uint32_t bits;
  memcpy(&bits, &value, 4);
  uint32_t sign = (bits >> 16) & 0x8000u;
  int32_t exp = (int32_t)((bits >> 23) & 0xffu);
  uint32_t mant = bits & 0x7fffffu;
  if (exp == 0xff)
    return (uint16_t)(sign | 0x7c00u | (mant ? 0x0200u : 0u));
  int32_t e = exp - 127;
  if (e >= 16)
    return (uint16_t)(sign | 0x7c00u);
  if (e >= -14) {
    uint32_t out = sign | ((uint32_t)(e + 15) << 10) | (mant >> 13);
    uint32_t rest = mant & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (out & 1u)))
      out += 1u; /* a carry into the exponent is the correct rounding */
    return (uint16_t)out;
  }
  if (e >= -25) {
    uint32_t full = mant | 0x800000u;
    uint32_t shift = (uint32_t)(-14 - e) + 13u;
    uint32_t m10 = full >> shift;
    uint32_t rest = full & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    uint32_t out = sign | m10;
    if (rest > half || (rest == half && (m10 & 1u)))
      out += 1u;
    return (uint16_t)out;
  }
  return (uint16_t)sign;
}

/* src/dtype.rs:87-106: binary16 -> f32 (exact). */
float ta_oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t mant = h & 0x3ffu;
  uint32_t out;
  if (exp == 0 && mant == 0) {
    out = sign;
  } else if (exp == 0) {
    int shift = 0;
    while (!(mant & 0x400u)) {
      mant <<= 1;
      ++shift;
    }
    mant &= 0x3ffu;
    out = sign | ((uint32_t)(127 - 15 - shift + 1) << 23) | (mant << 13);
  } else if (exp == 0x1f) {
    out = sign | 0x7f800000u | (mant ? (0x400000u | (mant << 13)) : 0u);
  } else {
    out = sign | ((exp + 127 - 15) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &out, 4);
  return f;
}

void ta_oracle_f32_to_f16_array(const float *src, uint16_t *dst, size_t len) {
  for (size_t i = 0; i < len; ++i)
    dst[i] = ta_oracle_f32_to_f16(src[i]);
}

void ta_oracle_f16_to_f32_array(const uint16_t *src, float *dst, size_t len) {
  for (size_t i = 0; i < len; ++i)
    dst[i] = ta_oracle_f16_to_f32(src[i]);
}

/* src/dtype.rs:110-112 applied elementwise, in place. */
void ta_oracle_round_via_f16(float *v, size_t len) {
  for (size_t i = 0; i < len; ++i)
    v[i] = ta_oracle_f16_to_f32(ta_oracle_f32_to_f16(v[i]));
}

/* src/matmul/api.rs:324-344: row-major [K, N] -> [N/tile][K][tile]. */
int ta_oracle_pack_row_tiles(const float *src, size_t k, size_t n,
                             size_t tile, float *dst) {
  if (tile == 0 || n % tile)
    return -1;
  size_t tiles = n / tile;
  for (size_t t = 0; t < tiles; ++t)
    for (size_t kk = 0; kk < k; ++kk)
      memcpy(dst + (t * k + kk) * tile, src + kk * n + t * tile,
             tile * sizeof(float));
  return 0;
}

/* tests/correctness/epilogue.rs:9-19 (cpu_activate), in double. */
static double activate(double x, uint32_t act) {
  switch (act) {
  case 1:
    return x > 0.0 ? x : 0.0;
  case 2:
    return x / (1.0 + exp(-x));
  case 3: {
    const double k0 = 0.7978845608028654;
    return 0.5 * x * (1.0 + tanh(k0 * (x + 0.044715 * x * x * x)));
  }
  default:
    return x;
  }
}

/* tests/correctness/epilogue.rs:24-47 (cpu_epilogue) in the order of
 * shaders/matmul_epilogue_common.glsl:14-21: +bias -> act -> binary with
 * D, in double, one f32 rounding at the end.  `c` holds batch planes of
 * m*n values that already include alpha and accumulate.  `bias` may be
 * null; bias_batch_stride is 0 for a shared [N] bias and N for [B, N].
 * binary: 0 none, 1 += beta*D, 2 *= D. */
void ta_oracle_epilogue(float *c, size_t total, uint32_t n, size_t mn,
                        const float *bias, uint32_t bias_batch_stride,
                        uint32_t act, uint32_t binary, const float *d,
                        float beta) {
  for (size_t i = 0; i < total; ++i) {
    size_t col = i % n, batch = i / mn;
    double x = (double)c[i];
    if (bias)
      x += (double)bias[batch * bias_batch_stride + col];
    x = activate(x, act);
    if (binary == 1)
      x += (double)beta * (double)d[i];
    else if (binary == 2)
      x *= (double)d[i];
    c[i] = (float)x;
  }
}

/* shaders/matmul_splitk2_kernel.glsl:138-142: split s of S owns
 * [k_lo, k_hi); the K % S remainder goes one each to the first splits. */
void ta_oracle_split_window(uint32_t k, uint32_t splits, uint32_t s,
                            uint32_t *k_lo, uint32_t *k_hi) {
  uint32_t per = k / splits, rem = k % splits;
  *k_lo = s * per + (s < rem ? s : rem);
  *k_hi = *k_lo + per + (s < rem ? 1u : 0u);
}
