// The device format encoders of csrc/l2c_formats.h built for the CPU, with
// row quantizers assembled from the same per-block functions the kernels
// call, so tests can compare every code, tie and block rule with the test
// oracle without a GPU (lib/libl2c_formats_host.so; not part of the library
// the applications link).
#include <cstddef>
#include <cstdint>

#pragma clang fp contract(off)
#include "../csrc/l2c_formats.h"

extern "C" {

// fmt: 0 E2M1, 1 E3M2, 2 UE4M3 / E4M3 (signed input allowed), 3 bf16 unused.
void l2cf_encode_array(int fmt, const float *v, size_t n, uint8_t *out) {
  for (size_t i = 0; i < n; ++i)
    out[i] = static_cast<uint8_t>(fmt == 0 ? l2c::e2m1_code(v[i]) : fmt == 1 ? l2c::e3m2_code(v[i])
                                                                            : l2c::e4m3_code(v[i]));
}

void l2cf_values(int fmt, float *out) {  // E2M1: 16 values, UE4M3: 128 values
  if (fmt == 0)
    for (unsigned c = 0; c < 16; ++c) out[c] = l2c::e2m1_value(c);
  else
    for (unsigned c = 0; c < 128; ++c) out[c] = l2c::ue4m3_value(c);
}

// Unpacked codes [rows][width] and scale codes, as the device quantizers
// compute them block by block.
void l2cf_quantize_mxfp6(const float *x, int rows, int width, uint8_t *codes, uint8_t *scales) {
  const long long blocks = static_cast<long long>(rows) * (width / 32);
  for (long long b = 0; b < blocks; ++b) {
    const float *v = x + 32 * b;
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = std::fmax(amax, std::fabs(v[i]));
    const int X = l2c::mxfp6_exponent(amax);
    const float inv = l2c::pow2_neg(X);
    for (int i = 0; i < 32; ++i) codes[32 * b + i] = amax > 0.0f ? static_cast<uint8_t>(l2c::e3m2_code(v[i] * inv)) : 0;
    scales[b] = amax > 0.0f ? static_cast<uint8_t>(X + 127) : 0;
  }
}

void l2cf_quantize_nvfp4(const float *x, int rows, int width, float s, uint8_t *codes, uint8_t *scales,
                         float *expanded) {
  const long long blocks = static_cast<long long>(rows) * (width / 16);
  for (long long b = 0; b < blocks; ++b) {
    const float *v = x + 16 * b;
    float amax = 0.0f;
    for (int i = 0; i < 16; ++i) amax = std::fmax(amax, std::fabs(v[i]));
    const unsigned sc = l2c::nvfp4_scale_code(amax, s);
    const float f = l2c::ue4m3_value(sc);
    for (int i = 0; i < 16; ++i) {
      const unsigned c = sc != 0 ? l2c::nvfp4_code(v[i], s, f) : 0u;
      codes[16 * b + i] = static_cast<uint8_t>(c);
      if (expanded) expanded[16 * b + i] = l2c::e2m1_value(c) * f;
    }
    scales[b] = static_cast<uint8_t>(sc);
  }
}

float l2cf_nvfp4_encode_scale(float amax) { return l2c::nvfp4_encode_scale(amax); }

}  // extern "C"
