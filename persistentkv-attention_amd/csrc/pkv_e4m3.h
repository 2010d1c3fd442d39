// pkv_e4m3.h — the OCP fp8 e4m3 encode of the KV append into fp8 pools (the bytes of
// torch's float8_e4m3fn cast), kept in one place for any kernel that stores fp8 K/V.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace pkv {

// OCP e4m3 byte of y: |y| clamped to 448, rounded to the nearest value with ties to the
// even code; NaN keeps its sign (0x7f / 0xff).
__device__ inline uint32_t e4m3_encode(float y) {
  const uint32_t sign = (__float_as_uint(y) >> 24) & 0x80u;
  if (y != y) return sign | 0x7Fu;
  const float a = fminf(fabsf(y), 448.0f);
  if (a < 0.015625f)  // below 2^-6: subnormal steps of 2^-9 (8 steps is the smallest normal)
    return sign | (uint32_t)__builtin_rintf(a * 512.0f);
  const uint32_t bits = __float_as_uint(a);
  int exponent = (int)(bits >> 23) - 127;  // -6 .. 8
  uint32_t mantissa = (bits >> 20) & 7u;
  const uint32_t rest = bits & 0xFFFFFu;   // the 20 mantissa bits below the kept 3
  if (rest > 0x80000u || (rest == 0x80000u && (mantissa & 1u))) ++mantissa;
  if (mantissa == 8u) {
    mantissa = 0;
    ++exponent;
  }
  return sign | ((uint32_t)(exponent + 7) << 3) | mantissa;
}

// Two 16-bit values (fp16, or bf16 when BF16_IN), low half first, to two e4m3 bytes of
// x / scale, low byte first.
template <bool BF16_IN>
__device__ inline float half_bits_to_float(uint32_t h) {
  if constexpr (BF16_IN) return __uint_as_float(h << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
template <bool BF16_IN>
__device__ inline uint32_t e4m3_pack2(uint32_t x2, float scale) {
  const uint32_t lo = e4m3_encode(half_bits_to_float<BF16_IN>(x2 & 0xFFFFu) / scale);
  const uint32_t hi = e4m3_encode(half_bits_to_float<BF16_IN>(x2 >> 16) / scale);
  return lo | (hi << 8);
}

}  // namespace pkv
