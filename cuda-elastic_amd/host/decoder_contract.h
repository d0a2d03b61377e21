// The contract check of the llama2c decoder (loom-private/llama2c-decoder),
// shared by the decoder application and the lowprec fp32 control, which must
// pass it unchanged: dimensions, the synthetic model, the expected tokens and
// dense double evaluation of probe sequences, and the three checks
// (applications/loom_private/decoder/oracle.cpp:1-230, contract.json
// "tolerances"). Also the RAII device and pinned arrays of both applications.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <memory>
#include <thread>
#include <vector>

#include "app_protocol.h"

namespace l2c_decoder {

struct Dims {
  long long batch, width, vocab, steps;
  size_t token_count() const { return static_cast<size_t>(batch * steps); }
  size_t activation_count() const { return static_cast<size_t>(steps * batch * width); }
  size_t row_count() const { return static_cast<size_t>(steps * batch * vocab); }
  // Offsets of (sequence, step) in the [steps][batch][...] diagnostics.
  size_t activation_at(long long b, long long s) const { return static_cast<size_t>((s * batch + b) * width); }
  size_t row_at(long long b, long long s) const { return static_cast<size_t>((s * batch + b) * vocab); }
};

// The synthetic model, evaluated from its definition (contract.json
// "data_generation"), never from device data.
struct SyntheticModel {
  long long vocab;
  double embedding(long long token, long long column) const { return column == token ? 4.0 : 1.0; }
  double norm_weight(long long) const { return 1.0; }
  double classifier(long long row, long long column) const {
    return column == (row + vocab - 1) % vocab ? 1.0 : 0.0;
  }
  long long prompt(long long sequence) const { return sequence % vocab; }
};

// Tolerances of the dense comparison (contract.json "tolerances").
constexpr double kActivationTolerance = 2.0e-6;  // normalized values and logits
constexpr double kProbabilityTolerance = 2.0e-5;
constexpr double kToleranceFloor = 1.0e-12;
constexpr int kReportLimit = 8;

// ---------------------------------------------------------------------------
// What the GPU must produce.

class Expectation {
 public:
  explicit Expectation(const Dims &dims) : dims_(dims), model_{dims.vocab} {
    // Every token follows t -> (t + 1) mod vocab from the prompt.
    tokens_.resize(dims.token_count());
    for (long long b = 0; b < dims.batch; ++b) {
      long long t = model_.prompt(b);
      for (long long s = 0; s < dims.steps; ++s) {
        t = (t + 1) % dims.vocab;
        tokens_[static_cast<size_t>(b * dims.steps + s)] = static_cast<int32_t>(t);
      }
    }
    // Probe sequences: up to 8, evenly spaced, first and last included.
    const long long n = std::min<long long>(8, dims.batch);
    for (long long i = 0; i < n; ++i) {
      const long long b = n == 1 ? 0 : i * (dims.batch - 1) / (n - 1);
      if (probes_.empty() || probes_.back() != b) probes_.push_back(b);
    }
    const size_t per_probe_w = static_cast<size_t>(dims.steps * dims.width);
    const size_t per_probe_v = static_cast<size_t>(dims.steps * dims.vocab);
    normalized_.assign(probes_.size() * per_probe_w, 0.0);
    logits_.assign(probes_.size() * per_probe_v, 0.0);
    probabilities_.assign(probes_.size() * per_probe_v, 0.0);
    std::vector<char> agrees(probes_.size(), 1);
    std::vector<std::thread> pool;
    for (size_t i = 0; i < probes_.size(); ++i)
      pool.emplace_back([&, i] {
        agrees[i] = dense_double(probes_[i], &normalized_[i * per_probe_w], &logits_[i * per_probe_v],
                                 &probabilities_[i * per_probe_v]);
      });
    for (auto &worker : pool) worker.join();
    consistent_ = std::all_of(agrees.begin(), agrees.end(), [](char ok) { return ok != 0; });
    if (!consistent_)
      std::fprintf(stderr, "decoder oracle: dense evaluation disagrees with the analytic token progression\n");
  }

  bool consistent() const { return consistent_; }
  int32_t token(long long b, long long s) const { return tokens_[static_cast<size_t>(b * dims_.steps + s)]; }
  const std::vector<long long> &probes() const { return probes_; }
  const double *normalized(size_t probe, long long s) const {
    return &normalized_[(probe * dims_.steps + s) * dims_.width];
  }
  const double *logits(size_t probe, long long s) const { return &logits_[(probe * dims_.steps + s) * dims_.vocab]; }
  const double *probabilities(size_t probe, long long s) const {
    return &probabilities_[(probe * dims_.steps + s) * dims_.vocab];
  }

 private:
  // Every step of one sequence in double, the classifier evaluated densely
  // (every row against every column). Returns whether the dense argmax
  // reproduces the analytic progression.
  bool dense_double(long long sequence, double *o_out, double *l_out, double *p_out) const {
    const long long W = dims_.width, V = dims_.vocab;
    std::vector<double> x(W), row(W);
    long long token = model_.prompt(sequence);
    bool agrees = true;
    for (long long s = 0; s < dims_.steps; ++s) {
      double *o = o_out + s * W, *l = l_out + s * V, *p = p_out + s * V;
      double squares = 0.0;
      for (long long j = 0; j < W; ++j) {
        x[j] = model_.embedding(token, j);
        squares += x[j] * x[j];
      }
      const double inv_rms = 1.0 / std::sqrt(squares / static_cast<double>(W) + 1.0e-5);
      for (long long j = 0; j < W; ++j) o[j] = model_.norm_weight(j) * (inv_rms * x[j]);
      for (long long r = 0; r < V; ++r) {
        for (long long j = 0; j < W; ++j) row[j] = model_.classifier(r, j);
        double acc = 0.0;
        for (long long j = 0; j < W; ++j) acc += row[j] * o[j];
        l[r] = acc;
      }
      const double top = *std::max_element(l, l + V);
      double z = 0.0;
      for (long long r = 0; r < V; ++r) z += (p[r] = std::exp(l[r] - top));
      long long argmax = 0;
      for (long long r = 0; r < V; ++r) {
        p[r] /= z;
        if (p[r] > p[argmax]) argmax = r;
      }
      agrees = agrees && argmax == (token + 1) % V;
      token = argmax;
    }
    return agrees;
  }

  Dims dims_;
  SyntheticModel model_;
  std::vector<int32_t> tokens_;
  std::vector<long long> probes_;
  std::vector<double> normalized_, logits_, probabilities_;
  bool consistent_ = true;
};

// Host copies of the device outputs.
struct HostView {
  const int32_t *tokens;       // [batch][steps]
  const float *normalized;     // [steps][batch][width]
  const float *logits;         // [steps][batch][vocab]
  const float *probabilities;  // [steps][batch][vocab]
};

// Within relative * |expected| + floor; NaN never is.
inline bool close(double observed, double expected, double relative) {
  return std::fabs(observed - expected) <= relative * std::fabs(expected) + kToleranceFloor;
}

// The three checks of the contract. The wording of every message matches the
// reference decoder's, which test scripts match on.
inline bool verify(const Dims &d, const Expectation &want, const HostView &got) {
  // 1. Every generated token, exactly.
  long long wrong_tokens = 0;
  for (long long b = 0; b < d.batch; ++b)
    for (long long s = 0; s < d.steps; ++s) {
      const int32_t actual = got.tokens[static_cast<size_t>(b * d.steps + s)];
      if (actual == want.token(b, s)) continue;
      if (wrong_tokens++ < kReportLimit)
        std::fprintf(stderr, "decoder: token mismatch sequence %lld step %lld: expected %d, actual %d\n", b, s,
                     want.token(b, s), actual);
    }

  // 2. Normalization invariants of every (sequence, step): the float mean of
  // squares and the float probability sum, both summed in double.
  const float square_tol = 2.0e-5f + 1.2e-7f * static_cast<float>(d.width);
  const float sum_tol = 1.0e-6f + 1.2e-7f * static_cast<float>(d.vocab);
  long long broken = 0;
  float square_seen = 0.0f, sum_seen = 0.0f;
  for (long long s = 0; s < d.steps; ++s)
    for (long long b = 0; b < d.batch; ++b) {
      const float *o = got.normalized + d.activation_at(b, s);
      const float *p = got.probabilities + d.row_at(b, s);
      double sq = 0.0, ps = 0.0;
      for (long long j = 0; j < d.width; ++j) sq += static_cast<double>(o[j]) * static_cast<double>(o[j]);
      for (long long r = 0; r < d.vocab; ++r) ps += static_cast<double>(p[r]);
      const float mean_square = static_cast<float>(sq / static_cast<double>(d.width));
      const float square_off = std::fabs(mean_square - 1.0f);
      const float sum_off = std::fabs(static_cast<float>(ps) - 1.0f);
      const bool square_ok = square_off <= square_tol, sum_ok = sum_off <= sum_tol;
      if (square_ok) square_seen = std::max(square_seen, square_off);
      if (sum_ok) sum_seen = std::max(sum_seen, sum_off);
      if (square_ok && sum_ok) continue;
      if (broken++ < kReportLimit)
        std::fprintf(stderr,
                     "decoder: invariant failure sequence %lld step %lld: mean square expected 1 +- %.3g, "
                     "actual %.9g; probability sum expected 1 +- %.3g, actual %.9g\n",
                     b, s, square_tol, mean_square, sum_tol, static_cast<float>(ps));
    }

  // 3. The probe sequences against the dense double evaluation.
  long long mismatches = 0;
  double seen[3] = {0.0, 0.0, 0.0};  // worst passing relative error per kind
  const char *const kinds[3] = {"normalized", "logit", "probability"};
  auto compare = [&](int kind, long long b, long long s, long long index, float actual, double expected,
                     double relative) {
    if (close(actual, expected, relative)) {
      seen[kind] = std::max(seen[kind], std::fabs(actual - expected) / std::max(std::fabs(expected), kToleranceFloor));
    } else if (mismatches++ < kReportLimit) {
      std::fprintf(stderr, "decoder: %s mismatch sequence %lld step %lld index %lld: expected %.9g, actual %.9g\n",
                   kinds[kind], b, s, index, expected, static_cast<double>(actual));
    }
  };
  for (size_t i = 0; i < want.probes().size(); ++i) {
    const long long b = want.probes()[i];
    for (long long s = 0; s < d.steps; ++s) {
      const float *o = got.normalized + d.activation_at(b, s);
      const float *l = got.logits + d.row_at(b, s);
      const float *p = got.probabilities + d.row_at(b, s);
      const double *eo = want.normalized(i, s), *el = want.logits(i, s), *ep = want.probabilities(i, s);
      for (long long j = 0; j < d.width; ++j) compare(0, b, s, j, o[j], eo[j], kActivationTolerance);
      for (long long r = 0; r < d.vocab; ++r) {
        compare(1, b, s, r, l[r], el[r], kActivationTolerance);
        compare(2, b, s, r, p[r], ep[r], kProbabilityTolerance);
      }
    }
  }

  const bool pass = want.consistent() && wrong_tokens == 0 && broken == 0 && mismatches == 0;
  std::fprintf(stderr,
               "decoder: %s: %lld/%lld tokens wrong; %lld/%lld (sequence, step) invariant failures (worst "
               "passing |mean square - 1| %.3g, |probability sum - 1| %.3g); dense check of %zu sequences x "
               "%lld steps: %lld mismatches (worst passing relative error normalized %.3g, logits %.3g, "
               "probabilities %.3g)\n",
               pass ? "PASS" : "FAIL", wrong_tokens, d.batch * d.steps, broken, d.batch * d.steps,
               static_cast<double>(square_seen), static_cast<double>(sum_seen), want.probes().size(), d.steps,
               mismatches, seen[0], seen[1], seen[2]);
  return pass;
}

// ---------------------------------------------------------------------------
// Device and pinned host memory owned by the workload.

struct HipFree {
  void operator()(void *p) const { (void)hipFree(p); }
};
struct HipHostFree {
  void operator()(void *p) const { (void)hipHostFree(p); }
};
template <typename T>
using DeviceArray = std::unique_ptr<T, HipFree>;
template <typename T>
using PinnedArray = std::unique_ptr<T, HipHostFree>;

template <typename T>
DeviceArray<T> device_array(size_t count) {
  void *p = nullptr;
  APP_HIP(hipMalloc(&p, count * sizeof(T)));
  return DeviceArray<T>(static_cast<T *>(p));
}
template <typename T>
PinnedArray<T> pinned_array(size_t count) {
  void *p = nullptr;
  APP_HIP(hipHostMalloc(&p, count * sizeof(T), hipHostMallocDefault));
  return PinnedArray<T>(static_cast<T *>(p));
}

}  // namespace l2c_decoder
