// Host reference of the lowprec classifier cases (see lowprec_reference.h).
#include "lowprec_reference.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>

#include "parallel.h"

namespace lowprec {

namespace {

int host_threads() {
  const unsigned n = std::thread::hardware_concurrency();
  return static_cast<int>(std::max(1u, std::min(16u, n)));
}

// Magnitudes of the non-negative codes, increasing with the code.
struct Table {
  std::vector<double> magnitude;
  unsigned sign_bit;  // 0: unsigned format
};

const Table &e2m1_table() {
  static const Table t = [] {
    Table r{{}, 8u};
    for (unsigned c = 0; c < 8; ++c) r.magnitude.push_back(c < 4 ? 0.5 * c : std::ldexp(2.0 + (c & 1u), (c >> 1) - 2));
    return r;
  }();
  return t;
}
const Table &e3m2_table() {
  static const Table t = [] {
    Table r{{}, 32u};
    for (unsigned c = 0; c < 32; ++c) {
      const int e = static_cast<int>(c >> 2), m = static_cast<int>(c & 3u);
      r.magnitude.push_back(e == 0 ? std::ldexp(m, -4) : std::ldexp(4.0 + m, e - 5));
    }
    return r;
  }();
  return t;
}
const Table &ue4m3_table() {
  static const Table t = [] {
    Table r{{}, 0u};
    for (unsigned c = 0; c < 127; ++c) {  // 0x7f is NaN
      const int e = static_cast<int>(c >> 3), m = static_cast<int>(c & 7u);
      r.magnitude.push_back(e == 0 ? std::ldexp(m, -9) : std::ldexp(8.0 + m, e - 10));
    }
    return r;
  }();
  return t;
}

// Nearest magnitude code by binary search; a midpoint goes to the even code;
// above the largest magnitude saturates.
unsigned nearest(const Table &t, double v) {
  const double a = std::fabs(v);
  const std::vector<double> &m = t.magnitude;
  const size_t hi = static_cast<size_t>(std::lower_bound(m.begin(), m.end(), a) - m.begin());
  unsigned code;
  if (hi == m.size()) {
    code = static_cast<unsigned>(m.size() - 1);
  } else if (hi == 0 || m[hi] == a) {
    code = static_cast<unsigned>(hi);
  } else {
    const double below = a - m[hi - 1], above = m[hi] - a;
    code = static_cast<unsigned>(below < above ? hi - 1 : above < below ? hi : ((hi - 1) % 2 == 0 ? hi - 1 : hi));
  }
  return (code != 0 && v < 0 && t.sign_bit) ? (code | t.sign_bit) : code;
}

double signed_value(const Table &t, unsigned code) {
  const unsigned mag = t.sign_bit ? code & (t.sign_bit - 1u) : code;
  const double v = t.magnitude[mag];
  return (t.sign_bit && (code & t.sign_bit)) ? -v : v;
}

}  // namespace

const char *case_name(int c) {
  static const char *const names[] = {"fp32", "bf16", "mxfp6", "nvfp4"};
  return c >= 0 && c < 4 ? names[c] : "?";
}

double e2m1_value(unsigned code) { return signed_value(e2m1_table(), code & 15u); }
double e3m2_value(unsigned code) { return signed_value(e3m2_table(), code & 63u); }
double ue4m3_value(unsigned code) { return ue4m3_table().magnitude[std::min(code & 127u, 126u)]; }
double ue8m0_value(unsigned code) { return std::ldexp(1.0, static_cast<int>(code) - 127); }
unsigned e2m1_encode(double v) { return nearest(e2m1_table(), v); }
unsigned e3m2_encode(double v) { return nearest(e3m2_table(), v); }
unsigned ue4m3_encode(double v) { return nearest(ue4m3_table(), v); }

double bf16_value(uint16_t bits) {
  const uint32_t wide = static_cast<uint32_t>(bits) << 16;
  float f;
  std::memcpy(&f, &wide, sizeof f);
  return f;
}

uint16_t bf16_encode(float v) {
  uint32_t bits;
  std::memcpy(&bits, &v, sizeof bits);
  const uint16_t down = static_cast<uint16_t>(bits >> 16);  // toward zero
  if ((bits & 0xffffu) == 0) return down;
  const uint16_t up = static_cast<uint16_t>(down + 1);  // next magnitude, same sign
  if ((up & 0x7f80u) == 0x7f80u) return down;           // never round a finite value to infinity
  const double dd = std::fabs(bf16_value(down) - v), du = std::fabs(bf16_value(up) - v);
  if (dd != du) return dd < du ? down : up;
  return (down & 1u) ? up : down;
}

Quantized quantize(int c, const float *x, long long rows, long long width) {
  Quantized q;
  q.codes.assign(static_cast<size_t>(rows * width), 0);
  if (c == kFp32) return q;
  const long long block = c == kMxfp6 ? 32 : 16;
  if (c != kBf16) q.scales.assign(static_cast<size_t>(rows * (width / block)), 0);
  float encode = 1.0f;
  if (c == kNvfp4) {
    float amax = 0.0f;
    for (long long i = 0; i < rows * width; ++i) amax = std::max(amax, std::fabs(x[i]));
    encode = amax > 0.0f ? 2688.0f / amax : 1.0f;
    q.decode = 1.0f / encode;
  }
  l2c_host::parallel_ranges(static_cast<size_t>(rows), host_threads(), [&](size_t r0, size_t r1, size_t) {
    for (long long r = static_cast<long long>(r0); r < static_cast<long long>(r1); ++r) {
      const float *row = x + r * width;
      uint16_t *codes = &q.codes[static_cast<size_t>(r * width)];
      if (c == kBf16) {
        for (long long k = 0; k < width; ++k) codes[k] = bf16_encode(row[k]);
        continue;
      }
      for (long long b = 0; b < width / block; ++b) {
        const float *v = row + b * block;
        float amax = 0.0f;
        for (long long i = 0; i < block; ++i) amax = std::max(amax, std::fabs(v[i]));
        uint8_t &scale = q.scales[static_cast<size_t>(r * (width / block) + b)];
        if (c == kMxfp6) {
          if (amax == 0.0f) continue;  // scale 0, codes 0
          int e;
          std::frexp(static_cast<double>(amax), &e);  // amax = f 2^e, f in [0.5, 1)
          const int shared = std::max(-127, std::min(127, e - 1 - 4));
          scale = static_cast<uint8_t>(shared + 127);
          for (long long i = 0; i < block; ++i)
            codes[b * block + i] = static_cast<uint16_t>(e3m2_encode(std::ldexp(static_cast<double>(v[i]), -shared)));
        } else {
          float target = amax / 6.0f;
          target = target * encode;
          const unsigned sc = ue4m3_encode(target);
          scale = static_cast<uint8_t>(sc);
          if (sc == 0) continue;
          const float f = static_cast<float>(ue4m3_value(sc));
          for (long long i = 0; i < block; ++i) {
            float t = v[i] * encode;
            t = t / f;
            codes[b * block + i] = static_cast<uint16_t>(e2m1_encode(t));
          }
        }
      }
    }
  });
  return q;
}

float dequantized(int c, const Quantized &q, long long width, long long r, long long k) {
  const uint16_t code = q.codes[static_cast<size_t>(r * width + k)];
  switch (c) {
    case kBf16: return static_cast<float>(bf16_value(code));
    case kMxfp6:
      return static_cast<float>(e3m2_value(code) * ue8m0_value(q.scales[static_cast<size_t>(r * (width / 32) + k / 32)]));
    case kNvfp4:
      return static_cast<float>(e2m1_value(code) * ue4m3_value(q.scales[static_cast<size_t>(r * (width / 16) + k / 16)]));
    default: return 0.0f;
  }
}

unsigned unpack_e3m2(const uint8_t *row, long long i) {
  const long long bit = 6 * i;
  unsigned window = row[bit / 8];
  if (bit % 8 > 2) window |= static_cast<unsigned>(row[bit / 8 + 1]) << 8;
  return (window >> (bit % 8)) & 63u;
}
unsigned unpack_e2m1(const uint8_t *row, long long i) { return (row[i / 2] >> (4 * (i % 2))) & 15u; }

namespace {

struct SplitMix64 {
  uint64_t state;
  uint64_t next() {
    uint64_t z = (state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  }
  double uniform() { return static_cast<double>(next() >> 11) * 0x1.0p-53; }
};

void normals(int seed, int stream, size_t count, float *out, float scale) {
  SplitMix64 g{static_cast<uint64_t>(seed) * 0x100000001b3ull + static_cast<uint64_t>(stream)};
  const double tau = 6.283185307179586476925286766559;
  for (size_t i = 0; i < count; i += 2) {
    const double u1 = g.uniform(), u2 = g.uniform();
    const double radius = std::sqrt(-2.0 * std::log(1.0 - u1));
    out[i] = static_cast<float>(radius * std::cos(tau * u2)) * scale;
    if (i + 1 < count) out[i + 1] = static_cast<float>(radius * std::sin(tau * u2)) * scale;
  }
}

}  // namespace

void fixture(int seed, long long width, long long vocab, float *embedding, float *classifier) {
  const size_t n = static_cast<size_t>(width * vocab);
  normals(seed, 1, n, embedding, 1.0f);
  normals(seed, 2, n, classifier, static_cast<float>(1.0 / std::sqrt(static_cast<double>(width))));
}

void rmsnorm_double(const float *x, long long width, double *out) {
  double squares = 0.0;
  for (long long j = 0; j < width; ++j) squares += static_cast<double>(x[j]) * x[j];
  const double scale = 1.0 / std::sqrt(squares / static_cast<double>(width) + static_cast<double>(1e-5f));
  for (long long j = 0; j < width; ++j) out[j] = scale * x[j];
}

void rmsnorm_float(const float *x, long long width, float *out) {
  float squares = 0.0f;
  for (long long j = 0; j < width; ++j) squares += x[j] * x[j];
  squares /= static_cast<float>(width);
  squares += 1e-5f;
  const float scale = 1.0f / std::sqrt(squares);
  for (long long j = 0; j < width; ++j) out[j] = 1.0f * (scale * x[j]);
}

void softmax_double(const double *logits, long long count, double *out) {
  double top = -INFINITY, sum = 0.0;
  for (long long r = 0; r < count; ++r) top = std::max(top, logits[r]);
  for (long long r = 0; r < count; ++r) sum += (out[r] = std::exp(logits[r] - top));
  for (long long r = 0; r < count; ++r) out[r] /= sum;
}

long long argmax_first(const double *values, long long count) {
  long long best = 0;
  for (long long r = 1; r < count; ++r)
    if (values[r] > values[best]) best = r;
  return best;
}

ErrorMetrics compare_logits(const std::vector<double> &reference, const std::vector<double> &actual, long long rows,
                            long long vocab) {
  ErrorMetrics m;
  m.rows = rows;
  double err2 = 0.0, ref2 = 0.0, variation = 0.0;
  std::vector<double> pr(static_cast<size_t>(vocab)), pa(static_cast<size_t>(vocab));
  for (long long b = 0; b < rows; ++b) {
    const double *ref = &reference[static_cast<size_t>(b * vocab)], *act = &actual[static_cast<size_t>(b * vocab)];
    for (long long r = 0; r < vocab; ++r) {
      const double e = act[r] - ref[r];
      m.max_abs_error = std::max(m.max_abs_error, std::fabs(e));
      err2 += e * e;
      ref2 += ref[r] * ref[r];
    }
    softmax_double(ref, vocab, pr.data());
    softmax_double(act, vocab, pa.data());
    double row = 0.0;
    for (long long r = 0; r < vocab; ++r) {
      const double d = std::fabs(pa[static_cast<size_t>(r)] - pr[static_cast<size_t>(r)]);
      m.max_abs_probability_error = std::max(m.max_abs_probability_error, d);
      row += d;
    }
    variation += 0.5 * row;
    m.top1_agree += argmax_first(ref, vocab) == argmax_first(act, vocab);
  }
  m.normalized_rms_error = ref2 > 0 ? std::sqrt(err2 / ref2) : 0.0;
  m.mean_total_variation = rows ? variation / static_cast<double>(rows) : 0.0;
  return m;
}

}  // namespace lowprec
