// Element and scale encoders of the low-precision formats, device side.
// Every encoder rounds to the nearest representable value with ties to the
// code whose least significant bit is 0, saturates at the largest magnitude,
// and returns +0 (code 0) for a magnitude that rounds to zero
// (experiments/blackwell/lowprec/spec.json "rounding"; the host reference
// reference.cpp:64-82 finds the same codes by table search).
//
// The functions are host and device code: lib/libl2c_formats_host.so builds
// them for the CPU so tests can compare them with the test oracle over every
// code and every tie.
#pragma once

#include <hip/hip_runtime.h>
#include <cmath>
#include <cstdint>

#define L2C_HD __host__ __device__ __forceinline__

namespace l2c {

L2C_HD unsigned f2u(float f) { return __builtin_bit_cast(unsigned, f); }
L2C_HD float u2f(unsigned u) { return __builtin_bit_cast(float, u); }

// E2M1: magnitudes {0, .5, 1, 1.5, 2, 3, 4, 6}, bit 3 the sign. The
// thresholds are the midpoints; a midpoint goes to the even code.
L2C_HD unsigned e2m1_code(float v) {
  const float t = fabsf(v);
  unsigned c;
  if (t <= 0.25f) c = 0;
  else if (t < 0.75f) c = 1;
  else if (t <= 1.25f) c = 2;
  else if (t < 1.75f) c = 3;
  else if (t <= 2.5f) c = 4;
  else if (t < 3.5f) c = 5;
  else if (t <= 5.0f) c = 6;
  else c = 7;
  return (c != 0 && v < 0.0f) ? (c | 8u) : c;
}

L2C_HD float e2m1_value(unsigned c) {
  const unsigned m = c & 7u;
  // 0, .5, 1, 1.5 are m / 2; 2, 3, 4, 6 are (2 + (m & 1)) * 2^((m >> 1) - 2) for m >= 4.
  const float mag = m < 4u ? 0.5f * static_cast<float>(m)
                           : static_cast<float>(2u + (m & 1u)) * static_cast<float>(1u << ((m >> 1) - 2u));
  return (c & 8u) ? -mag : mag;
}

// E4M3 (OCP, bias 7, largest 448 = 0x7e, 0x7f NaN never produced). With a
// non-negative argument this is UE4M3.
L2C_HD unsigned e4m3_code(float v) {
  const float a = fabsf(v);
  unsigned c;
  if (a < 0.015625f) {  // below 2^-6: subnormal codes m * 2^-9, m in 0..8
    c = static_cast<unsigned>(rintf(a * 512.0f));
  } else {
    const unsigned bits = f2u(a);
    int e = static_cast<int>((bits >> 23) & 0xffu) - 127;
    unsigned q = (bits >> 20) & 7u;
    const unsigned rem = bits & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) ++q;
    if (q == 8u) {
      q = 0;
      ++e;
    }
    c = e > 8 ? 0x7eu : ((static_cast<unsigned>(e + 7) << 3) | q);
    if (c > 0x7eu) c = 0x7eu;
  }
  return (c != 0 && v < 0.0f) ? (c | 0x80u) : c;
}

// Value of a UE4M3 code (bit 7 ignored): m * 2^-9, or (1 + m / 8) 2^(e - 7).
L2C_HD float ue4m3_value(unsigned c) {
  const unsigned e = (c >> 3) & 15u, m = c & 7u;
  return e == 0 ? static_cast<float>(m) * 0x1p-9f : u2f(((e + 120u) << 23) | (m << 20));
}

// E3M2 (bias 3, no infinities): subnormals m * 2^-4, largest 28 = 0x1f, bit 5
// the sign. A magnitude a < 28 in binade e = floor(log2 a) (>= -2) rounds to
// q = rint(a * 2^(2 - e)) in [4, 8], code ((e + 3) << 2) + q - 4, which
// carries into the next binade at q = 8; below 0.25 the step is 2^-4 and the
// code is rint(16 a) (rint ties to even, and the code's low bit is q's).
L2C_HD unsigned e3m2_code(float v) {
  const float a = fabsf(v);
  unsigned c;
  if (a >= 28.0f) {
    c = 31u;
  } else if (a < 0.25f) {
    c = static_cast<unsigned>(rintf(a * 16.0f));
  } else {
    const int e = static_cast<int>((f2u(a) >> 23) & 0xffu) - 127;  // -2 .. 4
    const float step_inv = u2f(static_cast<unsigned>(127 + 2 - e) << 23);
    const unsigned q = static_cast<unsigned>(rintf(a * step_inv));
    const unsigned code = (static_cast<unsigned>(e + 3) << 2) + q - 4u;
    c = code < 31u ? code : 31u;
  }
  return (c != 0 && v < 0.0f) ? (c | 32u) : c;
}

// MXFP6 block (spec.json "mxfp6"): for a block maximum a > 0 the shared
// exponent is X = floor(log2 a) - 4 from the exponent field, clamped below at
// -127 (subnormal maxima clamp too; the field tops out at 254, so X <= 123).
// Elements are E3M2(v * 2^-X): the power-of-two scaling is exact wherever
// the code can be nonzero. Scale code X + 127; a zero block has scale code 0.
L2C_HD int mxfp6_exponent(float amax) {
  const int x = static_cast<int>((f2u(amax) >> 23) & 0xffu) - 127 - 4;
  return x > -127 ? x : -127;
}
L2C_HD float pow2_neg(int x) { return u2f(static_cast<unsigned>(127 - x) << 23); }  // 2^-x, x in [-127, 123]

// NVFP4 block (spec.json "nvfp4"): scale code UE4M3((a / 6) * s) and element
// codes E2M1((v * s) / f), every step a float operation in this order (the
// callers compile with contraction off); scale code 0 zeroes the block.
L2C_HD unsigned nvfp4_scale_code(float amax, float s) {
  float target = amax / 6.0f;
  target = target * s;
  return e4m3_code(target);
}
L2C_HD unsigned nvfp4_code(float v, float s, float f) {
  float r = v * s;
  r = r / f;
  return e2m1_code(r);
}
L2C_HD float nvfp4_encode_scale(float tensor_amax) { return tensor_amax > 0.0f ? 2688.0f / tensor_amax : 1.0f; }

}  // namespace l2c
