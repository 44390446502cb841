// Scalar format conversions shared by the gfx950 kernels and the host-side
// exports. OCP e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa bits; no
// infinities; S.1111.111 is NaN; largest finite 448; subnormals k * 2^-9.
// All conversions round to nearest even, as torch's .to(float8_e4m3fn) and
// .to(bfloat16) do.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define NSSM_HD __host__ __device__ __forceinline__
#else
#define NSSM_HD static inline
#endif

NSSM_HD uint32_t nssm_f2u(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __float_as_uint(f);
#else
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
#endif
}

NSSM_HD float nssm_u2f(uint32_t u) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __uint_as_float(u);
#else
  float f;
  memcpy(&f, &u, 4);
  return f;
#endif
}

NSSM_HD float nssm_bf16_to_f32(uint16_t v) { return nssm_u2f((uint32_t)v << 16); }

NSSM_HD uint16_t nssm_f32_to_bf16(float f) {
  uint32_t u = nssm_f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Round-to-nearest-even float -> e4m3fn. Magnitudes that round above 448
// (>= 464) and NaN inputs give the NaN code, as torch's cast does.
NSSM_HD uint8_t nssm_f32_to_e4m3fn(float f) {
  const uint32_t u = nssm_f2u(f);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  const uint32_t au = u & 0x7fffffffu;
  if (au > 0x7f800000u) return (uint8_t)(sign | 0x7f);  // NaN
  if (au >= 0x3c800000u) {                              // |f| >= 2^-6: normal range
    // keep 3 mantissa bits, RNE on the 20 dropped bits; a carry bumps the exponent
    uint32_t r = au + 0x7ffffu + ((au >> 20) & 1u);
    int32_t e = (int32_t)(r >> 23) - 127 + 7;
    uint32_t m = (r >> 20) & 7u;
    if (e > 15 || (e == 15 && m == 7u)) return (uint8_t)(sign | 0x7f);  // overflow -> NaN
    return (uint8_t)(sign | (uint32_t)(e << 3) | m);
  }
  // subnormal range: value = k * 2^-9, k = rne(|f| * 512) in [0, 8]; k = 8 is 2^-6 (code 0x08)
  const float s = nssm_u2f(au) * 512.0f;  // exact: power-of-two scaling
  uint32_t k = (uint32_t)s;               // truncation
  const float frac = s - (float)k;
  if (frac > 0.5f || (frac == 0.5f && (k & 1u))) k += 1u;
  return (uint8_t)(sign | k);
}

NSSM_HD float nssm_e4m3fn_to_f32(uint8_t v) {
  const uint32_t sign = (uint32_t)(v & 0x80u) << 24;
  const uint32_t e = (v >> 3) & 15u, m = v & 7u;
  if (e == 15u && m == 7u) return nssm_u2f(sign | 0x7fc00000u);
  if (e == 0u) {
    const float s = (float)m * 0.001953125f;  // m * 2^-9, exact
    return sign ? -s : s;
  }
  return nssm_u2f(sign | ((e + 120u) << 23) | (m << 20));
}
