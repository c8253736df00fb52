// f32 <-> f16 host conversion and the packed row-tile layout.
#include <cstring>

#include "internal.hpp"

namespace tensor_ash {

uint64_t dtype_size(DType d) { return d == DType::F32 ? 4 : 2; }
const char *dtype_name(DType d) { return d == DType::F32 ? "f32" : "f16"; }

// src/dtype.rs:42-84: round to nearest even; overflow -> signed inf; NaN
// keeps a quiet payload bit; underflow -> signed zero.
uint16_t f32_to_f16_bits(float value) {
  uint32_t bits;
  std::memcpy(&bits, &value, 4);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const int32_t exp = (int32_t)((bits >> 23) & 0xffu);
  const uint32_t mant = bits & 0x7fffffu;
  if (exp == 0xff)
    return (uint16_t)(sign | 0x7c00u | (mant ? 0x0200u : 0u));
  const int32_t e = exp - 127;
  if (e >= 16)
    return (uint16_t)(sign | 0x7c00u);
  if (e >= -14) {
    uint32_t out = sign | ((uint32_t)(e + 15) << 10) | (mant >> 13);
    const uint32_t rest = mant & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (out & 1u)))
      ++out; // a carry into the exponent is still the correct rounding
    return (uint16_t)out;
  }
  if (e >= -25) {
    const uint32_t full = mant | 0x800000u;
    const uint32_t shift = (uint32_t)(-14 - e) + 13u;
    const uint32_t m10 = full >> shift;
    const uint32_t rest = full & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    uint32_t out = sign | m10;
    if (rest > half || (rest == half && (m10 & 1u)))
      ++out;
    return (uint16_t)out;
  }
  return (uint16_t)sign;
}

// src/dtype.rs:87-106, except that subnormal halves decode to their exact
// value (the reference's subnormal branch yields half of it).
float f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
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
    out = sign | ((uint32_t)(127 - 15 + 1 - shift) << 23) | ((mant & 0x3ffu) << 13);
  } else if (exp == 0x1f) {
    out = sign | 0x7f800000u | (mant ? (0x400000u | (mant << 13)) : 0u);
  } else {
    out = sign | ((exp + 127 - 15) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &out, 4);
  return f;
}

float round_f32_via_f16(float value) { return f16_bits_to_f32(f32_to_f16_bits(value)); }

// src/matmul/api.rs:324-344.
std::vector<float> pack_f16w_row_tiles(const float *src, size_t k, size_t n, size_t tile_n) {
  if (tile_n == 0 || n % tile_n != 0)
    fail("N=" + std::to_string(n) + " is not a multiple of tile_n=" + std::to_string(tile_n));
  std::vector<float> out(k * n);
  const size_t tiles = n / tile_n;
  for (size_t t = 0; t < tiles; ++t)
    for (size_t kk = 0; kk < k; ++kk)
      std::memcpy(&out[(t * k + kk) * tile_n], &src[kk * n + t * tile_n], tile_n * sizeof(float));
  return out;
}

// Packing tile for the decode GEMV: 64-column tiles whenever N allows
// (one 128-byte f16 row per tile row, 256 contiguous bytes per wave
// load), else 32.  The reference's NVIDIA-tuned k16/k16_v2 split
// (src/pipeline/routing.rs:10-23) is not reproduced; callers that pack
// with this function always match the kernel that reads the layout.
uint32_t f16w_row_tile_n(uint32_t /*k*/, uint32_t n) { return n % 64 == 0 ? 64 : 32; }

} // namespace tensor_ash
