// Host reference of the lowprec classifier cases, independent of the device
// encoders: every code is found by searching the format's value table (the
// device computes codes with bit arithmetic), in double. It is what the
// application's implementation check and self-test compare the device with
// (experiments/blackwell/lowprec/spec.json "formats", "rounding", "mxfp6",
// "nvfp4", "fixtures", "implementation_check", "accuracy"; the reference's
// own host reference is reference.h / reference.cpp of that directory).
#pragma once

#include <cstdint>
#include <vector>

namespace lowprec {

enum Case { kFp32 = 0, kBf16 = 1, kMxfp6 = 2, kNvfp4 = 3 };
const char *case_name(int c);

// Value of a code: E2M1 (bit 3 sign), E3M2 (bit 5 sign), UE4M3, UE8M0.
double e2m1_value(unsigned code);
double e3m2_value(unsigned code);
double ue4m3_value(unsigned code);
double ue8m0_value(unsigned code);
// Nearest code, ties to the code whose lowest bit is 0, saturating, +0 for a
// magnitude that rounds to zero. ue4m3 takes non-negative values.
unsigned e2m1_encode(double v);
unsigned e3m2_encode(double v);
unsigned ue4m3_encode(double v);
// bf16 bits, nearest with ties to even, by comparing the two neighbours.
uint16_t bf16_encode(float v);
double bf16_value(uint16_t bits);

// One [rows][width] matrix quantized the way a case converts it, unpacked:
// codes one per value (bf16 bits for kBf16), scales one per block
// ([rows][width / 32] MXFP6, [rows][width / 16] NVFP4), decode = d of NVFP4.
struct Quantized {
  std::vector<uint16_t> codes;
  std::vector<uint8_t> scales;
  float decode = 1.0f;
};
Quantized quantize(int lowprec_case, const float *x, long long rows, long long width);
// The value of element k of row r without the NVFP4 tensor decode scale
// (which joins alpha); exact in float for every case.
float dequantized(int lowprec_case, const Quantized &q, long long width, long long r, long long k);

// Unpacking of the device layouts: value i of a packed row.
unsigned unpack_e3m2(const uint8_t *row, long long i);
unsigned unpack_e2m1(const uint8_t *row, long long i);

// Dense fixture: vocab x width embedding (standard normals of stream 1) and
// classifier (stream 2 times float(1 / sqrt(width))), splitmix64 seeded with
// seed * 0x100000001b3 + stream, Box-Muller in double from consecutive pairs.
void fixture(int seed, long long width, long long vocab, float *embedding, float *classifier);

// rmsnorm with weight 1: in double, and in float with a sequential square sum.
void rmsnorm_double(const float *x, long long width, double *out);
void rmsnorm_float(const float *x, long long width, float *out);
void softmax_double(const double *logits, long long count, double *out);
long long argmax_first(const double *values, long long count);

struct ErrorMetrics {
  long long rows = 0, top1_agree = 0;
  double max_abs_error = 0, normalized_rms_error = 0, max_abs_probability_error = 0, mean_total_variation = 0;
};
// Case logits against reference logits, both [rows][vocab].
ErrorMetrics compare_logits(const std::vector<double> &reference, const std::vector<double> &actual, long long rows,
                            long long vocab);

}  // namespace lowprec
