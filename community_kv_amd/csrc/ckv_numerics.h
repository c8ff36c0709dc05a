// Scalar numerics shared by the HIP kernels and the host-side numerics probe.
//
// Everything here is a fixed sequence of IEEE round-to-nearest-even fp32
// operations and integer bit manipulation, so that the CPU oracle
// (oracle/numerics.py) reproduces it bit for bit.  The library is compiled with
// -ffp-contract=off: no multiply-add pair is fused.
//
//   ckv_f32_to_f16_bits   fp32 -> IEEE half bits, round to nearest even
//   ckv_ordered_key16     order-preserving key of half bits (reference
//                         descriptor_selection.cu:30-33)
//   ckv_f32_to_bf16_bits  fp32 -> bf16 bits, round to nearest even
//   ckv_f32_to_e4m3       fp32 -> OCP E4M3 ("fn"), clamp to +-448 then round to
//                         nearest even (reference graph/partition.py:452-454)
//   ckv_expf, ckv_logf    Cody-Waite reduced exp with a degree-7 Taylor
//                         polynomial; log via 2*atanh((m-1)/(m+1)).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define CKV_HD __host__ __device__ inline
#else
#define CKV_HD static inline
#endif

CKV_HD uint32_t ckv_f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
CKV_HD float ckv_u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

CKV_HD uint16_t ckv_f32_to_f16_bits(float f) {
  const uint32_t x = ckv_f2u(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t a = x & 0x7fffffffu;
  if (a >= 0x7f800000u) return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // >= 65520 rounds to inf
  if (a >= 0x38800000u) {                                   // normal half
    const uint32_t r = a + 0xfffu + ((a >> 13) & 1u);
    return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
  }
  if (a <= 0x33000000u) return (uint16_t)sign;  // <= 2^-25 rounds to zero
  const uint32_t e = a >> 23;
  const uint32_t m = (a & 0x7fffffu) | 0x800000u;
  const uint32_t s = 126u - e;  // quanta of 2^-24
  uint32_t q = m >> s;
  const uint32_t rem = m & ((1u << s) - 1u);
  const uint32_t half = 1u << (s - 1u);
  if (rem > half || (rem == half && (q & 1u))) ++q;
  return (uint16_t)(sign | q);
}

CKV_HD uint16_t ckv_ordered_key16(uint16_t bits) {
  return (uint16_t)(bits ^ ((bits & 0x8000u) ? 0xffffu : 0x8000u));
}

CKV_HD uint16_t ckv_f32_to_bf16_bits(float f) {
  const uint32_t x = ckv_f2u(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(((x | 0x00400000u) >> 16) & 0xffffu);
  const uint32_t r = x + 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(r >> 16);
}

CKV_HD float ckv_bf16_to_f32(uint16_t b) { return ckv_u2f(((uint32_t)b) << 16); }

CKV_HD uint8_t ckv_f32_to_e4m3(float f) {
  const uint32_t x = ckv_f2u(f);
  const uint32_t sign = (x >> 24) & 0x80u;
  const uint32_t a = x & 0x7fffffffu;
  if (a > 0x7f800000u) return 0x7fu;                      // NaN
  if (a >= 0x43e00000u) return (uint8_t)(sign | 0x7eu);   // clamp to 448
  if (a >= 0x3c800000u) {                                 // normal (>= 2^-6)
    const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
    return (uint8_t)(sign | ((r - 0x3c000000u) >> 20));
  }
  if (a <= 0x3a800000u) return (uint8_t)sign;             // <= 2^-10 rounds to zero
  const uint32_t e = a >> 23;
  const uint32_t m = (a & 0x7fffffu) | 0x800000u;
  const uint32_t s = 141u - e;                            // quanta of 2^-9
  uint32_t q = m >> s;
  const uint32_t rem = m & ((1u << s) - 1u);
  const uint32_t half = 1u << (s - 1u);
  if (rem > half || (rem == half && (q & 1u))) ++q;
  return (uint8_t)(sign | q);
}

CKV_HD float ckv_e4m3_to_f32(uint8_t c) {
  const uint32_t sign = ((uint32_t)(c & 0x80u)) << 24;
  const uint32_t e = (c >> 3) & 0xfu;
  const uint32_t m = c & 0x7u;
  if (e == 0xfu && m == 0x7u) return ckv_u2f(0x7fc00000u | sign);
  if (e == 0u) {
    const float v = (float)m * 0.001953125f;  // m * 2^-9, exact
    return (c & 0x80u) ? -v : v;
  }
  return ckv_u2f(sign | ((e + 120u) << 23) | (m << 20));
}

#define CKV_LOG2E 1.44269504088896340736f
#define CKV_LN2_HI 0.693145751953125f
#define CKV_LN2_LO 1.42860682030941723212e-6f
#define CKV_SQRT2 1.41421356237309504880f

CKV_HD float ckv_rint(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_rintf(x);
#else
  return __builtin_rintf(x);
#endif
}

// exp(x): n = rint(x*log2e); r = (x - n*ln2_hi) - n*ln2_lo; Taylor degree 7 in
// Horner form; result p * 2^n.  Results below 2^-125 are flushed to zero.
CKV_HD float ckv_expf(float x) {
  if (x != x) return x;
  const uint32_t ux = ckv_f2u(x);
  if (ux == 0xff800000u) return 0.0f;
  if (ux == 0x7f800000u) return x;
  const float t = x * CKV_LOG2E;
  float n = ckv_rint(t);
  if (n < -200.0f) n = -200.0f;
  if (n > 200.0f) n = 200.0f;
  float r = x - n * CKV_LN2_HI;
  r = r - n * CKV_LN2_LO;
  float p = 1.0f / 5040.0f;
  p = p * r + 1.0f / 720.0f;
  p = p * r + 1.0f / 120.0f;
  p = p * r + 1.0f / 24.0f;
  p = p * r + 1.0f / 6.0f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  const int ni = (int)n;
  if (ni < -125) return 0.0f;
  if (ni > 127) return ckv_u2f(0x7f800000u);
  return p * ckv_u2f(((uint32_t)(ni + 127)) << 23);
}

// log(x) for positive normal x.
CKV_HD float ckv_logf(float x) {
  if (x != x || x < 0.0f) return ckv_u2f(0x7fc00000u);
  if (x == 0.0f) return ckv_u2f(0xff800000u);
  const uint32_t bits = ckv_f2u(x);
  if (bits == 0x7f800000u) return x;
  int e = (int)((bits >> 23) & 0xffu) - 127;
  float m = ckv_u2f((bits & 0x007fffffu) | 0x3f800000u);
  if (m > CKV_SQRT2) {
    m = m * 0.5f;
    e += 1;
  }
  const float f = m - 1.0f;
  const float s = f / (m + 1.0f);
  const float s2 = s * s;
  float p = 2.0f / 11.0f;
  p = p * s2 + 2.0f / 9.0f;
  p = p * s2 + 2.0f / 7.0f;
  p = p * s2 + 2.0f / 5.0f;
  p = p * s2 + 2.0f / 3.0f;
  p = p * s2 + 2.0f;
  const float logm = s * p;
  const float ef = (float)e;
  return ef * CKV_LN2_HI + (ef * CKV_LN2_LO + logm);
}
