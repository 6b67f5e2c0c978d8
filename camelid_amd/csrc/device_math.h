// device_math.h -- scalar numerics shared by the HIP kernels and host code.
//
// Every function here reproduces, bit for bit, the f32 arithmetic Camelid's CPU
// path performs, so kernels built on them can be bit-exact:
//   * f16 conversions: the reference's own bit algorithm (inference.rs:20767-20830).
//   * expf: glibc 2.35's x86-64 expf (the FMA ifunc variant), which is what Rust's
//     f32::exp calls on Linux.  It is NOT correctly rounded (about 1.7e5 of the 2^32
//     inputs are 1 ulp off), so a correctly rounded exp would not match.  The method
//     is the published ARM optimized-routines expf (2017, MIT): x*N/ln2 = k + r with
//     N = 32, a 32-entry table of 2^(i/32) and a cubic in r, evaluated in binary64.
//     The table entries are the correctly rounded binary64 values of 2^(i/32) (with the
//     index folded out of the exponent field); the range reduction and the cubic use
//     fused multiply-adds exactly where glibc's FMA build contracts them.  Checked
//     against glibc on a dense sample on the host (tests/test_abi_and_seam.py) and on
//     all 2^32 inputs on the device (tests/test_gpu_kernels.py).
//   * quantize_q8_0_block: inference.rs:16953-16971.
#pragma once
#include <stdint.h>
#include <string.h>
#include <math.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define CM_HD __host__ __device__ __forceinline__
#else
#define CM_HD inline
#endif

namespace cm {

CM_HD uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
CM_HD float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
CM_HD uint64_t d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
CM_HD double u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

// f32 -> f16 bits, round to nearest even; NaN -> canonical 0x7e00 (inference.rs:20767).
CM_HD uint16_t f32_to_f16_bits(float value) {
  uint32_t bits = f2u(value);
  uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  int32_t e = (int32_t)((bits >> 23) & 0xffu);
  uint32_t mant = bits & 0x007fffffu;
  if (e == 0xff) return (uint16_t)(sign | (mant == 0 ? 0x7c00u : 0x7e00u));
  int32_t he = e - 112;  // e - 127 + 15
  if (he >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (he <= 0) {
    if (he < -10) return sign;
    uint32_t m = mant | 0x00800000u;
    uint32_t shift = (uint32_t)(14 - he);
    uint32_t hm = m >> shift;
    uint32_t rb = 1u << (shift - 1);
    if ((m & rb) != 0 && ((m & (rb - 1)) != 0 || (hm & 1u) != 0)) hm += 1;
    return (uint16_t)(sign | hm);
  }
  uint32_t half = (uint32_t)sign | ((uint32_t)he << 10) | (mant >> 13);
  if ((mant & 0x1000u) != 0 && ((mant & 0x0fffu) != 0 || (half & 1u) != 0)) half += 1;
  return (uint16_t)half;
}

// f16 bits -> f32, exact (inference.rs:20803).
CM_HD float f16_bits_to_f32(uint16_t bits) {
  uint32_t sign = ((uint32_t)(bits & 0x8000u)) << 16;
  uint32_t e = (bits & 0x7c00u) >> 10;
  uint32_t frac = bits & 0x03ffu;
  uint32_t out;
  if (e == 0) {
    if (frac == 0) {
      out = sign;
    } else {
      // subnormal half: value = frac * 2^-24, normalised
      int32_t lz = 0;
      uint32_t m = frac;
      while ((m & 0x0400u) == 0) { m <<= 1; ++lz; }
      out = sign | ((uint32_t)(127 - 14 - lz) << 23) | ((m & 0x03ffu) << 13);
    }
  } else if (e == 0x1f) {
    out = sign | 0x7f800000u | (frac << 13);
  } else {
    out = sign | ((e + 112u) << 23) | (frac << 13);
  }
  return u2f(out);
}

// constexpr at namespace scope: usable from both host and device code.
constexpr uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

// glibc-identical expf (see the header comment).
// tab: kExp2Tab or a copy of it (the decode attention keeps one in LDS)
CM_HD float glibc_expf_t(float x, const uint64_t* tab) {
  const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
  const double kShift = 0x1.8p+52;
  const double C0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
  const double C1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
  const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  uint32_t ux = f2u(x);
  uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {                 // |x| >= 88 or NaN
    if (ux == 0xff800000u) return 0.0f;   // -inf
    if (abstop >= 0x7f8u) return x + x;   // +inf or NaN
    if (x > 0x1.62e42ep6f) return u2f(0x7f800000u);  // overflow
    if (x < -0x1.9fe368p6f) return 0.0f;             // underflow
  }
  double xd = (double)x;
  double kd = fma(kInvLn2N, xd, kShift);
  uint64_t ki = d2u(kd);
  kd -= kShift;
  double r = fma(kInvLn2N, xd, -kd);
  uint64_t t = tab[ki & 31u] + (ki << 47);
  double s = u2d(t);
  double z = fma(C0, r, C1);
  double r2 = r * r;
  double y = fma(C2, r, 1.0);
  y = fma(z, r2, y);
  y = y * s;
  return (float)y;
}

CM_HD float glibc_expf(float x) { return glibc_expf_t(x, kExp2Tab); }

// Q8_0 block quantizer (inference.rs:16953-16971): amax fold, scale = f16(amax/127),
// quants from the UNROUNDED inverse, round half away from zero, clamp [-128, 127].
// Returns the f16-valued scale as f32.
CM_HD float quantize_q8_0_block(const float* v, int8_t* q) {
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  float unrounded = amax / 127.0f;
  float scale = f16_bits_to_f32(f32_to_f16_bits(unrounded));
  float inv = unrounded == 0.0f ? 0.0f : 1.0f / unrounded;
  for (int i = 0; i < 32; ++i) {
    float r = roundf(v[i] * inv);
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    q[i] = (int8_t)r;
  }
  return scale;
}

// SwiGLU element (tensor/mod.rs:1943-1967): (g / (1 + exp(-g))) * u.
CM_HD float silu_mul1(float g, float u) { return (g / (1.0f + glibc_expf(-g))) * u; }

}  // namespace cm
