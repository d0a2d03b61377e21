// Thin extern "C" driver over the reference's own host code, compiled from
// the reference tree as it lies (never copied): llama2c/llama2c_common.h and
// experiments/blackwell/lowprec/reference.cpp. Built by oracle/Makefile into
// oracle/_ref/libl2c_ref.so. TEST INFRASTRUCTURE ONLY: tests use it to pin
// the oracle's restatement; nothing in the product loads it.
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "llama2c_common.h"
#include "reference.h"

extern "C" {

float ref_uniform(uint64_t seed, uint64_t stream, uint64_t index) {
  return llama2c_uniform(seed, stream, index);
}

double ref_gamma(int n) { return llama2c_gamma_probabilistic(n); }

// mode 0 deterministic, 1 random (the only modes the reference has).
void ref_fill(int mode, uint64_t seed, int batch, int size, int rows, float *input,
              float *probabilities, float *weight, float *matrix) {
  InputOptions o;
  o.random = mode != 0;
  o.seed = mode != 0 ? seed : 0;
  std::vector<float> in, pr, w, m;
  fill_inputs(o, batch, size, rows, &in, &pr, &w, &m);
  std::memcpy(input, in.data(), in.size() * 4);
  std::memcpy(probabilities, pr.data(), pr.size() * 4);
  std::memcpy(weight, w.data(), w.size() * 4);
  std::memcpy(matrix, m.data(), m.size() * 4);
}

// validate_all of the reference on given outputs; tolerance / reference
// receive the per-row arrays. Returns 1 when valid.
int ref_validate_all(int mode, uint64_t seed, const float *input, const float *probabilities,
                     const float *weight, const float *matrix, const float *normalized,
                     const float *softmax, const float *product, int batch, int size, int rows,
                     float *tolerance, double *reference) {
  InputOptions o;
  o.random = mode != 0;
  o.seed = seed;
  const size_t n = static_cast<size_t>(batch) * size, m = static_cast<size_t>(rows) * size;
  std::vector<float> tol;
  std::vector<double> ref;
  const bool valid = validate_all(
      o, std::vector<float>(input, input + n), std::vector<float>(probabilities, probabilities + n),
      std::vector<float>(weight, weight + size), std::vector<float>(matrix, matrix + m),
      std::vector<float>(normalized, normalized + n), std::vector<float>(softmax, softmax + n),
      std::vector<float>(product, product + rows), batch, size, rows, &tol, &ref);
  std::memcpy(tolerance, tol.data(), tol.size() * 4);
  std::memcpy(reference, ref.data(), ref.size() * 8);
  return valid ? 1 : 0;
}

int ref_write_dump(const char *path, int mode, uint64_t seed, int batch, int size, int rows,
                   const float *normalized, const float *softmax, const float *product,
                   const float *tolerance, const double *reference) {
  InputOptions o;
  o.random = mode != 0;
  o.seed = seed;
  return write_dump(path, o, batch, size, rows, normalized, softmax, product,
                    std::vector<float>(tolerance, tolerance + rows),
                    std::vector<double>(reference, reference + rows))
             ? 1
             : 0;
}

// lowprec formats: 0 E2M1, 1 E3M2, 2 UE4M3, 3 UE8M0.
unsigned ref_encode(int format, double v) {
  return lowprec_ref::encode(static_cast<lowprec_ref::Format>(format), v);
}
double ref_decode(int format, unsigned code) {
  return lowprec_ref::decode(static_cast<lowprec_ref::Format>(format), code);
}
uint16_t ref_to_bf16(float v) { return lowprec_ref::to_bf16(v); }

// The first `count` standard normals of stream 1 (the fixture embedding).
void ref_normals_stream1(int seed, long long count, float *out) {
  const lowprec_ref::Fixture f = lowprec_ref::make_fixture(seed, count, 1);
  std::memcpy(out, f.embedding.data(), static_cast<size_t>(count) * 4);
}

}  // extern "C"

extern "C" {

void ref_uniform_array(uint64_t seed, uint64_t stream, uint64_t start, size_t n, float *out) {
  for (size_t i = 0; i < n; ++i) out[i] = llama2c_uniform(seed, stream, start + i);
}

void ref_encode_array(int format, const double *v, size_t n, uint8_t *out) {
  for (size_t i = 0; i < n; ++i)
    out[i] = static_cast<uint8_t>(lowprec_ref::encode(static_cast<lowprec_ref::Format>(format), v[i]));
}

void ref_to_bf16_array(const float *v, size_t n, uint16_t *out) {
  for (size_t i = 0; i < n; ++i) out[i] = lowprec_ref::to_bf16(v[i]);
}

// The reference's MXFP6 / NVFP4 quantizers (experiments/blackwell/lowprec/reference.cpp).
void ref_quantize_mxfp6(const float *X, int rows, int width, uint8_t *codes, uint8_t *scales) {
  for (int r = 0; r < rows; ++r)
    lowprec_ref::quantize_mxfp6(X + static_cast<size_t>(r) * width, width, codes + static_cast<size_t>(r) * width,
                                scales + static_cast<size_t>(r) * (width / 32));
}
void ref_quantize_nvfp4(const float *X, int rows, int width, float s, uint8_t *codes, uint8_t *scales) {
  for (int r = 0; r < rows; ++r)
    lowprec_ref::quantize_nvfp4(X + static_cast<size_t>(r) * width, width, s, codes + static_cast<size_t>(r) * width,
                                scales + static_cast<size_t>(r) * (width / 16));
}
float ref_nvfp4_encode_scale(float amax) { return lowprec_ref::nvfp4_encode_scale(amax); }
float ref_nvfp4_decode_scale(float s) { return lowprec_ref::nvfp4_decode_scale(s); }
// Values i of packed rows.
unsigned ref_unpack_e3m2(const uint8_t *row, long long i) { return lowprec_ref::unpack_e3m2(row, i); }
unsigned ref_unpack_e2m1(const uint8_t *row, long long i) { return lowprec_ref::unpack_e2m1(row, i); }

}  // extern "C"
