// The lowprec decoder classifier experiment on MI355X: the llama2c decoder
// (loom-private/llama2c-decoder) with only its dense classifier replaced by
// a BF16, MXFP6 or NVFP4 contraction, under the loom_private protocol, plus
// the specification's self-test and accuracy modes.
//
// What it must do is fixed by experiments/blackwell/lowprec (spec.json: cases,
// formats, checks, metrics; decoder_lowprec.cu: the workload, its checks and
// modes; README.md). Per step: l2c_decoder_rmsnorm -> the case's activation
// conversion -> the case's classifier -> l2c_decoder_softmax_argmax with the
// token fed back on the device. Weights are converted once at setup.
//   fp32   l2c_matmul (the decoder's classifier, fp32 matrix cores)
//   bf16   l2c_to_bf16_x4 -> l2c_matmul_bf16
//   mxfp6  l2c_quantize_mxfp6 -> l2c_matmul_mxfp6 (scaled matrix cores)
//   nvfp4  l2c_nvfp4_tensor_scales (s, d, alpha) -> l2c_quantize_nvfp4 (codes,
//          scales and the exact bf16 expansion) -> l2c_matmul_bf16 with alpha
//          read from device memory
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "../../include/l2c.h"
#include "../../include/l2c_harness.h"
#include "decoder_contract.h"
#include "lowprec_reference.h"
#include "app_protocol.h"
#include "parallel.h"

namespace {

using l2c_decoder::DeviceArray;
using l2c_decoder::device_array;
using l2c_decoder::PinnedArray;
using l2c_decoder::pinned_array;
using namespace lowprec;

constexpr long long kLargeBatch = 1024, kLargeWidth = 16384, kLargeVocab = 8192, kLargeSteps = 4;
constexpr long long kFixtureBatch = 64, kFixtureWidth = 1024, kFixtureVocab = 128;
constexpr double kDeviceLimitGiB = 64.0;
// sha256 of experiments/blackwell/lowprec/spec.json, the specification this
// application implements (recorded in every result).
constexpr const char *kSpecSha256 = "1a56ed12366829cbf1b952d99267143f4d74f64411858cb6e7748e389616a64c";
constexpr int kReportLimit = 5;

int threads() { return static_cast<int>(std::max(1u, std::min(16u, std::thread::hardware_concurrency()))); }

// The converted form of one [rows][width] operand on the device.
struct Operand {
  long long rows = 0, width = 0;
  DeviceArray<uint8_t> codes;    // MXFP6: 3 bytes per 4 values; NVFP4: 1 per 2
  DeviceArray<uint8_t> scales;   // one byte per block, [rows][width / block]
  DeviceArray<uint16_t> wide;    // bf16 values (BF16) or the NVFP4 bf16 expansion
  DeviceArray<float> tensor;     // NVFP4: s, d
  size_t code_bytes = 0, scale_bytes = 0, wide_count = 0;
};

class LowprecWorkload final : public appproto::Application {
 public:
  LowprecWorkload(int lowprec_case, long long batch, long long width, long long vocab, long long steps, int fixture,
                  int fault = 0)
      : c_(lowprec_case), d_{batch, width, vocab, steps}, fixture_(fixture), fault_(fault) {}

  appproto::AppInfo info() const override {
    using appproto::Json;
    appproto::AppInfo i;
    i.identity = std::string("blackwell-experiments/lowprec-decoder-classifier/") + case_name(c_);
    i.dimensions.add("batch", Json::whole(d_.batch))
        .add("width", Json::whole(d_.width))
        .add("vocab", Json::whole(d_.vocab))
        .add("steps", Json::whole(d_.steps))
        .add("fixture", Json::whole(fixture_))
        .add("case", Json::text(case_name(c_)))
        .add("generated_tokens", Json::whole(d_.batch * d_.steps))
        .add("classifier_macs_per_step", Json::whole(d_.batch * d_.vocab * d_.width));
    i.application_scope =
        "prompt upload (pinned H2D), token reset, every step (rmsnorm, activation conversion with scale "
        "generation, classifier contraction, softmax+argmax with on-device token feedback), generated-token "
        "download; converted weights resident from setup";
    i.compute_scope =
        "token reset and every step (rmsnorm, activation conversion, classifier contraction, softmax+argmax)";
    return i;
  }

  long long batch() const { return d_.batch; }
  long long width() const { return d_.width; }
  long long vocab() const { return d_.vocab; }
  long long steps() const { return d_.steps; }
  const std::vector<float> &host_embedding() const { return host_embedding_; }
  const std::vector<float> &host_classifier() const { return host_classifier_; }
  float *normalized(long long s) const { return normalized_.get() + d_.activation_at(0, s); }
  float *logits(long long s) const { return logits_.get() + d_.row_at(0, s); }
  const int *generated() const { return host_generated_.get(); }
  void download_outputs(float *normalized_out, float *logits_out, float *probabilities_out) const {
    APP_HIP(hipMemcpy(normalized_out, normalized_.get(), d_.activation_count() * 4, hipMemcpyDeviceToHost));
    APP_HIP(hipMemcpy(logits_out, logits_.get(), d_.row_count() * 4, hipMemcpyDeviceToHost));
    APP_HIP(hipMemcpy(probabilities_out, probabilities_.get(), d_.row_count() * 4, hipMemcpyDeviceToHost));
  }

  void prepare(hipStream_t stream) override {
    const size_t model_count = static_cast<size_t>(d_.vocab * d_.width);
    embedding_ = device_array<float>(model_count);
    classifier_ = device_array<float>(model_count);
    norm_weight_ = device_array<float>(static_cast<size_t>(d_.width));
    prompts_ = device_array<int>(static_cast<size_t>(d_.batch));
    tokens_ = device_array<int>(static_cast<size_t>(d_.batch));
    generated_ = device_array<int>(d_.token_count());
    normalized_ = device_array<float>(d_.activation_count());
    logits_ = device_array<float>(d_.row_count());
    probabilities_ = device_array<float>(d_.row_count());
    partials_ = device_array<float>(L2C_NVFP4_PARTIALS);
    host_prompts_ = pinned_array<int>(static_cast<size_t>(d_.batch));
    host_generated_ = pinned_array<int>(d_.token_count());
    if (fixture_ == 0) {
      APP_L2C(l2c_decoder_init_model(embedding_.get(), classifier_.get(), norm_weight_.get(),
                                    static_cast<int>(d_.width), static_cast<int>(d_.vocab), stream));
    } else {
      host_embedding_.resize(model_count);
      host_classifier_.resize(model_count);
      lowprec::fixture(fixture_, d_.width, d_.vocab, host_embedding_.data(), host_classifier_.data());
      const std::vector<float> ones(static_cast<size_t>(d_.width), 1.0f);
      APP_HIP(hipMemcpyAsync(embedding_.get(), host_embedding_.data(), model_count * 4, hipMemcpyHostToDevice, stream));
      APP_HIP(hipMemcpyAsync(classifier_.get(), host_classifier_.data(), model_count * 4, hipMemcpyHostToDevice, stream));
      APP_HIP(hipMemcpyAsync(norm_weight_.get(), ones.data(), ones.size() * 4, hipMemcpyHostToDevice, stream));
      APP_HIP(hipStreamSynchronize(stream));
    }
    for (long long b = 0; b < d_.batch; ++b) host_prompts_.get()[b] = static_cast<int>(b % d_.vocab);
    if (c_ != kFp32) {
      weights_ = make_operand(d_.vocab);
      for (long long s = 0; s < d_.steps; ++s) activations_.push_back(make_operand(d_.batch));
      if (c_ == kNvfp4) alpha_ = device_array<float>(static_cast<size_t>(d_.steps));
    }
    APP_HIP(hipStreamSynchronize(stream));
    hipEvent_t start, stop;
    APP_HIP(hipEventCreate(&start));
    APP_HIP(hipEventCreate(&stop));
    APP_HIP(hipEventRecord(start, stream));
    convert_weights(stream);
    APP_HIP(hipEventRecord(stop, stream));
    APP_HIP(hipEventSynchronize(stop));
    float ms = 0.0f;
    APP_HIP(hipEventElapsedTime(&ms, start, stop));
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
    std::fprintf(stderr, "%s: case %s, fixture %d, weight conversion %.3f ms (setup)\n", appproto::program(),
                 case_name(c_), fixture_, static_cast<double>(ms));
  }

  void enqueue(appproto::Scope scope, hipStream_t stream) override {
    const bool whole = scope == appproto::Scope::kApplication;
    if (whole)
      APP_HIP(hipMemcpyAsync(prompts_.get(), host_prompts_.get(), static_cast<size_t>(d_.batch) * sizeof(int),
                             hipMemcpyHostToDevice, stream));
    enqueue_steps(stream);
    if (whole)
      APP_HIP(hipMemcpyAsync(host_generated_.get(), generated_.get(), d_.token_count() * sizeof(int),
                             hipMemcpyDeviceToHost, stream));
  }

  void enqueue_steps(hipStream_t stream) {
    APP_HIP(hipMemcpyAsync(tokens_.get(), prompts_.get(), static_cast<size_t>(d_.batch) * sizeof(int),
                          hipMemcpyDeviceToDevice, stream));
    const int B = static_cast<int>(d_.batch), W = static_cast<int>(d_.width), V = static_cast<int>(d_.vocab),
              S = static_cast<int>(d_.steps);
    for (int s = 0; s < S; ++s) {
      APP_L2C(l2c_decoder_rmsnorm(normalized(s), tokens_.get(), embedding_.get(), norm_weight_.get(), W, V, B, stream));
      enqueue_classifier(s, stream);
      APP_L2C(l2c_decoder_softmax_argmax(probabilities_.get() + d_.row_at(0, s), logits(s), tokens_.get(),
                                        generated_.get(), V, B, S, s, stream));
    }
  }

  // The classifier of step s on whatever normalized(s) holds.
  void enqueue_classifier(int s, hipStream_t stream) {
    const int B = static_cast<int>(d_.batch), W = static_cast<int>(d_.width), V = static_cast<int>(d_.vocab);
    if (c_ == kFp32) {
      APP_L2C(l2c_matmul(logits(s), normalized(s), classifier_.get(), B, W, V, stream));
      return;
    }
    Operand &a = activations_[static_cast<size_t>(s)];
    convert(normalized(s), a, alpha_ ? alpha_.get() + s : nullptr, stream);
    if (c_ == kMxfp6)
      APP_L2C(l2c_matmul_mxfp6(logits(s), a.codes.get(), a.scales.get(), weights_.codes.get(), weights_.scales.get(), B,
                              W, V, stream));
    else
      APP_L2C(l2c_matmul_bf16(logits(s), a.wide.get(), weights_.wide.get(), c_ == kNvfp4 ? alpha_.get() + s : nullptr,
                             B, W, V, stream));
  }

  void convert_weights(hipStream_t stream) {
    if (c_ != kFp32) convert(classifier_.get(), weights_, nullptr, stream);
  }

  void scramble_outputs(hipStream_t stream) override {
    auto poison = [&](void *p, size_t bytes) {
      if (p && bytes) APP_HIP(hipMemsetAsync(p, 0xFF, bytes, stream));
    };
    poison(prompts_.get(), static_cast<size_t>(d_.batch) * sizeof(int));
    poison(tokens_.get(), static_cast<size_t>(d_.batch) * sizeof(int));
    poison(generated_.get(), d_.token_count() * sizeof(int));
    poison(normalized_.get(), d_.activation_count() * sizeof(float));
    poison(logits_.get(), d_.row_count() * sizeof(float));
    poison(probabilities_.get(), d_.row_count() * sizeof(float));
    for (Operand &a : activations_) {
      poison(a.codes.get(), a.code_bytes);
      poison(a.scales.get(), a.scale_bytes);
      poison(a.wide.get(), a.wide_count * 2);
      poison(a.tensor.get(), 8);
    }
    if (alpha_) poison(alpha_.get(), static_cast<size_t>(d_.steps) * 4);
    std::memset(host_generated_.get(), 0xFF, d_.token_count() * sizeof(int));
  }

  void derive_expected() override {
    if (c_ != kFp32) {
      APP_HIP(hipDeviceSynchronize());
      const std::vector<float> w = host_weights();
      const Quantized expected = quantize(c_, w.data(), d_.vocab, d_.width);
      const Quantized actual = download(weights_);
      weights_match_ = compare("weights", expected, actual, d_.vocab);
      dequantized_weights_.resize(w.size());
      l2c_host::parallel_ranges(static_cast<size_t>(d_.vocab), threads(), [&](size_t r0, size_t r1, size_t) {
        for (long long r = static_cast<long long>(r0); r < static_cast<long long>(r1); ++r)
          for (long long k = 0; k < d_.width; ++k)
            dequantized_weights_[static_cast<size_t>(r * d_.width + k)] = dequantized(c_, expected, d_.width, r, k);
      });
      weight_decode_ = expected.decode;
    }
    if (c_ == kFp32 && fixture_ == 0) contract_ = std::make_unique<l2c_decoder::Expectation>(d_);
  }

  bool outputs_match() override {
    download_diagnostics();
    if (fault_ == 3) {
      // Logits as a contraction that ignored alpha would leave them.
      for (float &l : host_logits_) l /= alpha_host_;
    }
    return implementation_check();
  }

  uint64_t outputs_digest() const override {
    appproto::Digest h;
    h.add(host_generated_.get(), d_.token_count() * sizeof(int))
        .add(host_normalized_.data(), host_normalized_.size() * 4)
        .add(host_logits_.data(), host_logits_.size() * 4)
        .add(host_probabilities_.data(), host_probabilities_.size() * 4);
    for (const std::vector<uint8_t> &bytes : host_activation_bytes_) h.add(bytes.data(), bytes.size());
    return h.value();
  }

  // Self-test: the device conversion of a [rows][width] matrix against the host
  // reference (NVFP4 also alpha = d * 0.75).
  bool selftest(const std::vector<float> &m, long long rows) {
    if (c_ == kFp32) return true;
    DeviceArray<float> dm = device_array<float>(m.size());
    APP_HIP(hipMemcpy(dm.get(), m.data(), m.size() * 4, hipMemcpyHostToDevice));
    Operand o = make_operand(rows);
    DeviceArray<float> other = device_array<float>(1), alpha = device_array<float>(1);
    const float three_quarters = 0.75f;
    APP_HIP(hipMemcpy(other.get(), &three_quarters, 4, hipMemcpyHostToDevice));
    other_decode_override_ = other.get();
    convert(dm.get(), o, alpha.get(), nullptr);
    other_decode_override_ = nullptr;
    APP_HIP(hipDeviceSynchronize());
    const Quantized expected = quantize(c_, m.data(), rows, d_.width);
    bool pass = compare("self-test", expected, download(o), rows);
    if (c_ == kNvfp4) {
      float got = 0.0f;
      APP_HIP(hipMemcpy(&got, alpha.get(), 4, hipMemcpyDeviceToHost));
      const float want = expected.decode * three_quarters;
      if (got != want) {
        std::fprintf(stderr, "%s: self-test alpha %.9g, expected %.9g\n", appproto::program(),
                     static_cast<double>(got), static_cast<double>(want));
        pass = false;
      }
    }
    return pass;
  }

 private:
  // Test hook (--set fault=N, check only), the reference's mutant classes
  // planted in the downloaded step-0 activations instead of the kernels:
  // 1 an element code one step toward zero (rounding), 2 two neighbouring
  // block scales exchanged (scale layout); 3 (after the download) the logits
  // divided by alpha, as a contraction that ignored alpha would leave them.
  void plant(Quantized &q) const {
    if (fault_ == 1) {
      for (uint16_t &code : q.codes) {
        const unsigned mag = c_ == kBf16 ? code & 0x7fffu : c_ == kMxfp6 ? code & 31u : code & 7u;
        if (mag > 1) {
          --code;
          return;
        }
      }
    } else if (fault_ == 2) {
      for (size_t i = 0; i + 1 < q.scales.size(); i += 2)
        if (q.scales[i] != q.scales[i + 1]) {
          std::swap(q.scales[i], q.scales[i + 1]);
          return;
        }
    }
  }

  Operand make_operand(long long rows) {
    Operand o;
    o.rows = rows;
    o.width = d_.width;
    const size_t n = static_cast<size_t>(rows * d_.width);
    if (c_ == kBf16 || c_ == kNvfp4) {
      o.wide_count = n;
      o.wide = device_array<uint16_t>(n);
    }
    if (c_ == kMxfp6) {
      APP_L2C(l2c_mxfp6_bytes(static_cast<int>(rows), static_cast<int>(d_.width), &o.code_bytes, &o.scale_bytes));
    } else if (c_ == kNvfp4) {
      o.code_bytes = n / 2;
      o.scale_bytes = n / 16;
      o.tensor = device_array<float>(2);
    }
    if (o.code_bytes) o.codes = device_array<uint8_t>(o.code_bytes);
    if (o.scale_bytes) o.scales = device_array<uint8_t>(o.scale_bytes);
    return o;
  }

  // FP32 [rows][width] at x -> operand o. NVFP4 activations (alpha given) get
  // alpha = d_activations * d_weights.
  void convert(const float *x, Operand &o, float *alpha, hipStream_t stream) {
    const int rows = static_cast<int>(o.rows), W = static_cast<int>(d_.width);
    const long long n = o.rows * d_.width;
    switch (c_) {
      case kBf16: APP_L2C(l2c_to_bf16_x4(o.wide.get(), x, n, stream)); break;
      case kMxfp6: APP_L2C(l2c_quantize_mxfp6(o.codes.get(), o.scales.get(), x, rows, W, stream)); break;
      case kNvfp4: {
        const float *other = alpha ? (other_decode_override_ ? other_decode_override_ : weights_.tensor.get() + 1)
                                   : nullptr;
        APP_L2C(l2c_nvfp4_tensor_scales(o.tensor.get(), alpha, other, x, n, partials_.get(), stream));
        APP_L2C(l2c_quantize_nvfp4(o.codes.get(), o.scales.get(), o.wide.get(), x, o.tensor.get(), rows, W, stream));
        break;
      }
      default: break;
    }
  }

  std::vector<float> host_weights() const {
    if (fixture_ != 0) return host_classifier_;
    std::vector<float> w(static_cast<size_t>(d_.vocab * d_.width), 0.0f);
    for (long long r = 0; r < d_.vocab; ++r) w[static_cast<size_t>(r * d_.width + (r + d_.vocab - 1) % d_.vocab)] = 1.0f;
    return w;
  }

  // Downloads and unpacks an operand.
  Quantized download(const Operand &o) const {
    Quantized q;
    const size_t n = static_cast<size_t>(o.rows * d_.width);
    q.codes.resize(n);
    if (c_ == kBf16) {
      APP_HIP(hipMemcpy(q.codes.data(), o.wide.get(), n * 2, hipMemcpyDeviceToHost));
      return q;
    }
    std::vector<uint8_t> bytes(o.code_bytes), scale_bytes(o.scale_bytes);
    APP_HIP(hipMemcpy(bytes.data(), o.codes.get(), o.code_bytes, hipMemcpyDeviceToHost));
    APP_HIP(hipMemcpy(scale_bytes.data(), o.scales.get(), o.scale_bytes, hipMemcpyDeviceToHost));
    const long long W = d_.width;
    q.scales.resize(static_cast<size_t>(o.rows * (W / (c_ == kMxfp6 ? 32 : 16))));
    if (c_ == kMxfp6) {
      // Tiled operand layout: codes [W/128][Rp/32][4][32][24 B], scales [W/128][Rp][4].
      const long long Rp = (o.rows + 31) / 32 * 32;
      l2c_host::parallel_ranges(static_cast<size_t>(o.rows), threads(), [&](size_t r0, size_t r1, size_t) {
        for (long long r = static_cast<long long>(r0); r < static_cast<long long>(r1); ++r)
          for (long long kb = 0; kb < W / 32; ++kb) {
            const long long t = kb / 4, b = kb % 4;
            const uint8_t *block = bytes.data() + (((t * (Rp / 32) + r / 32) * 4 + b) * 32 + r % 32) * 24;
            for (long long j = 0; j < 32; ++j)
              q.codes[static_cast<size_t>(r * W + kb * 32 + j)] = static_cast<uint16_t>(unpack_e3m2(block, j));
            q.scales[static_cast<size_t>(r * (W / 32) + kb)] = scale_bytes[static_cast<size_t>((t * Rp + r) * 4 + b)];
          }
      });
    } else {
      q.scales = scale_bytes;
      l2c_host::parallel_ranges(static_cast<size_t>(o.rows), threads(), [&](size_t r0, size_t r1, size_t) {
        for (long long r = static_cast<long long>(r0); r < static_cast<long long>(r1); ++r)
          for (long long k = 0; k < W; ++k)
            q.codes[static_cast<size_t>(r * W + k)] = static_cast<uint16_t>(unpack_e2m1(bytes.data() + r * (W / 2), k));
      });
    }
    if (c_ == kNvfp4) {
      float ts[2];
      APP_HIP(hipMemcpy(ts, o.tensor.get(), 8, hipMemcpyDeviceToHost));
      q.decode = ts[1];
      // The bf16 expansion the contraction multiplies must be the exact value
      // of every code and scale.
      std::vector<uint16_t> wide(n);
      APP_HIP(hipMemcpy(wide.data(), o.wide.get(), n * 2, hipMemcpyDeviceToHost));
      long long bad = 0;
      for (size_t i = 0; i < n; ++i) {
        const long long r = static_cast<long long>(i) / d_.width, k = static_cast<long long>(i) % d_.width;
        if (bf16_value(wide[i]) != static_cast<double>(dequantized(c_, q, d_.width, r, k))) ++bad;
      }
      if (bad) {
        std::fprintf(stderr, "%s: %lld bf16 expansion values differ from their codes\n", appproto::program(), bad);
        q.decode = NAN;  // fails the comparison
      }
    }
    return q;
  }

  bool compare(const char *what, const Quantized &expected, const Quantized &actual, long long rows) const {
    long long code_errors = 0, scale_errors = 0;
    const char *app = appproto::program();
    for (size_t i = 0; i < expected.codes.size(); ++i)
      if (expected.codes[i] != actual.codes[i] && code_errors++ < kReportLimit)
        std::fprintf(stderr, "%s: %s code mismatch row %lld column %lld: expected 0x%x, actual 0x%x\n", app, what,
                     static_cast<long long>(i) / d_.width, static_cast<long long>(i) % d_.width, expected.codes[i],
                     actual.codes[i]);
    for (size_t i = 0; i < expected.scales.size(); ++i)
      if (expected.scales[i] != actual.scales[i] && scale_errors++ < kReportLimit)
        std::fprintf(stderr, "%s: %s scale mismatch block %zu: expected 0x%x, actual 0x%x\n", app, what, i,
                     expected.scales[i], actual.scales[i]);
    const bool decode_ok = expected.decode == actual.decode;
    if (!decode_ok)
      std::fprintf(stderr, "%s: %s tensor decode scale %.9g, expected %.9g\n", app, what,
                   static_cast<double>(actual.decode), static_cast<double>(expected.decode));
    std::fprintf(stderr, "%s: %s (%lld rows): %lld code and %lld scale mismatches\n", app, what, rows, code_errors,
                 scale_errors);
    return code_errors == 0 && scale_errors == 0 && decode_ok;
  }

  void download_diagnostics() {
    host_normalized_.resize(d_.activation_count());
    host_logits_.resize(d_.row_count());
    host_probabilities_.resize(d_.row_count());
    APP_HIP(hipMemcpy(host_normalized_.data(), normalized_.get(), host_normalized_.size() * 4, hipMemcpyDeviceToHost));
    APP_HIP(hipMemcpy(host_logits_.data(), logits_.get(), host_logits_.size() * 4, hipMemcpyDeviceToHost));
    APP_HIP(hipMemcpy(host_probabilities_.data(), probabilities_.get(), host_probabilities_.size() * 4,
                     hipMemcpyDeviceToHost));
    host_activation_bytes_.clear();
    for (const Operand &a : activations_) {
      std::vector<uint8_t> bytes(a.code_bytes + a.scale_bytes + a.wide_count * 2 + (a.tensor ? 8 : 0));
      uint8_t *p = bytes.data();
      if (a.code_bytes) APP_HIP(hipMemcpy(p, a.codes.get(), a.code_bytes, hipMemcpyDeviceToHost));
      p += a.code_bytes;
      if (a.scale_bytes) APP_HIP(hipMemcpy(p, a.scales.get(), a.scale_bytes, hipMemcpyDeviceToHost));
      p += a.scale_bytes;
      if (a.wide_count) APP_HIP(hipMemcpy(p, a.wide.get(), a.wide_count * 2, hipMemcpyDeviceToHost));
      p += a.wide_count * 2;
      if (a.tensor) APP_HIP(hipMemcpy(p, a.tensor.get(), 8, hipMemcpyDeviceToHost));
      host_activation_bytes_.push_back(std::move(bytes));
    }
  }

  const float *embedding_row(long long token, std::vector<float> &scratch) const {
    if (fixture_ != 0) return &host_embedding_[static_cast<size_t>(token * d_.width)];
    scratch.assign(static_cast<size_t>(d_.width), 1.0f);
    scratch[static_cast<size_t>(token)] = 4.0f;
    return scratch.data();
  }

  // spec.json "implementation_check": every stage against an independent host
  // computation from the GPU's own inputs to that stage.
  bool implementation_check() {
    const char *app = appproto::program();
    const long long B = d_.batch, W = d_.width, V = d_.vocab, S = d_.steps;
    // 1. Normalized rows against rmsnorm in double of the token the GPU fed back.
    std::atomic<int> reported{0};
    auto report = [&]() { return reported.fetch_add(1) < kReportLimit; };
    std::vector<long long> norm_errors(static_cast<size_t>(S * B), 0), range_errors(static_cast<size_t>(S * B), 0);
    l2c_host::parallel_ranges(static_cast<size_t>(S * B), threads(), [&](size_t j0, size_t j1, size_t) {
      std::vector<double> row(static_cast<size_t>(W));
      std::vector<float> scratch;
      for (size_t job = j0; job < j1; ++job) {
        const long long s = static_cast<long long>(job) / B, b = static_cast<long long>(job) % B;
        const long long token = s == 0 ? host_prompts_.get()[b] : host_generated_.get()[b * S + s - 1];
        if (token < 0 || token >= V) {
          range_errors[job] = 1;
          continue;
        }
        rmsnorm_double(embedding_row(token, scratch), W, row.data());
        const float *o = &host_normalized_[d_.activation_at(b, s)];
        for (long long k = 0; k < W; ++k) {
          const double e = row[static_cast<size_t>(k)];
          if (!(std::fabs(o[k] - e) <= 2e-6 * std::fabs(e) + 1e-12)) {
            if (norm_errors[job]++ == 0 && report())
              std::fprintf(stderr, "%s: normalized mismatch step %lld sequence %lld column %lld: expected %.9g, "
                           "actual %.9g\n", app, s, b, k, e, static_cast<double>(o[k]));
          }
        }
      }
    });
    long long normalized_errors = 0, token_range_errors = 0;
    for (size_t i = 0; i < norm_errors.size(); ++i) normalized_errors += norm_errors[i], token_range_errors += range_errors[i];

    // 2. Converted activations, bit for bit, every step (and NVFP4 alpha).
    bool activations_ok = true;
    std::vector<std::vector<float>> act(static_cast<size_t>(S));
    std::vector<float> alpha(static_cast<size_t>(S), 1.0f);
    if (c_ != kFp32) {
      for (long long s = 0; s < S; ++s) {
        const Quantized expected = quantize(c_, &host_normalized_[d_.activation_at(0, s)], B, W);
        char what[48];
        std::snprintf(what, sizeof what, "activations step %lld", s);
        Quantized actual = download(activations_[static_cast<size_t>(s)]);
        if (s == 0) plant(actual);
        activations_ok = compare(what, expected, actual, B) && activations_ok;
        std::vector<float> &a = act[static_cast<size_t>(s)];
        a.resize(static_cast<size_t>(B * W));
        for (long long b = 0; b < B; ++b)
          for (long long k = 0; k < W; ++k) a[static_cast<size_t>(b * W + k)] = dequantized(c_, expected, W, b, k);
        if (c_ == kNvfp4) {
          alpha[static_cast<size_t>(s)] = expected.decode * weight_decode_;
          if (s == 0) alpha_host_ = alpha[0];
          float got = 0.0f;
          APP_HIP(hipMemcpy(&got, alpha_.get() + s, 4, hipMemcpyDeviceToHost));
          if (got != alpha[static_cast<size_t>(s)]) {
            std::fprintf(stderr, "%s: alpha step %lld %.9g, expected %.9g\n", app, s, static_cast<double>(got),
                         static_cast<double>(alpha[static_cast<size_t>(s)]));
            activations_ok = false;
          }
        }
      }
    }

    // 3. Logits of up to 8 sequences, every step and row, against the double
    // product of the operands the GPU multiplied; the bound holds for FP32
    // accumulation in any order.
    std::vector<long long> sampled;
    const long long count = std::min<long long>(8, B);
    for (long long i = 0; i < count; ++i) sampled.push_back(count == 1 ? 0 : i * (B - 1) / (count - 1));
    const double u = 0x1p-23, gamma = static_cast<double>(W) * u / (1.0 - static_cast<double>(W) * u);
    const std::vector<float> fp32_weights = c_ == kFp32 ? host_weights() : std::vector<float>();
    const std::vector<float> &weights = c_ == kFp32 ? fp32_weights : dequantized_weights_;
    std::vector<long long> logit_errors(static_cast<size_t>(count * S), 0);
    std::vector<double> worst(static_cast<size_t>(count * S), 0.0);
    l2c_host::parallel_ranges(static_cast<size_t>(count * S), threads(), [&](size_t j0, size_t j1, size_t) {
      for (size_t job = j0; job < j1; ++job) {
        const long long i = static_cast<long long>(job) / S, s = static_cast<long long>(job) % S;
        const long long b = sampled[static_cast<size_t>(i)];
        const float *a = c_ == kFp32 ? &host_normalized_[d_.activation_at(b, s)] : &act[static_cast<size_t>(s)][static_cast<size_t>(b * W)];
        const double scale = alpha[static_cast<size_t>(s)];
        for (long long r = 0; r < V; ++r) {
          const float *w = &weights[static_cast<size_t>(r * W)];
          double sum = 0.0, mag = 0.0;
          for (long long k = 0; k < W; ++k) {
            const double p = static_cast<double>(a[k]) * static_cast<double>(w[k]);
            sum += p;
            mag += std::fabs(p);
          }
          const double expected = sum * scale;
          const double actual = host_logits_[d_.row_at(b, s) + static_cast<size_t>(r)];
          const double bound = gamma * mag * std::fabs(scale) + u * std::fabs(expected) + 1e-30;
          const double error = std::fabs(actual - expected);
          if (!(error <= bound)) {
            if (logit_errors[job]++ == 0)
              std::fprintf(stderr, "%s: logit mismatch step %lld sequence %lld row %lld: expected %.9g, actual %.9g, "
                           "bound %.3g\n", app, s, b, r, expected, actual, bound);
          } else if (mag > 0) {
            worst[job] = std::max(worst[job], error / (mag * std::fabs(scale)));
          }
        }
      }
    });
    long long total_logit_errors = 0;
    double worst_logit = 0.0;
    for (size_t j = 0; j < logit_errors.size(); ++j) total_logit_errors += logit_errors[j], worst_logit = std::max(worst_logit, worst[j]);

    // 4. Probabilities and tokens from the GPU's own logits.
    std::vector<long long> prob_errors(static_cast<size_t>(S * B), 0), tok_errors(static_cast<size_t>(S * B), 0);
    l2c_host::parallel_ranges(static_cast<size_t>(S * B), threads(), [&](size_t j0, size_t j1, size_t) {
      std::vector<double> l(static_cast<size_t>(V)), p(static_cast<size_t>(V));
      for (size_t job = j0; job < j1; ++job) {
        const long long s = static_cast<long long>(job) / B, b = static_cast<long long>(job) % B;
        const float *gl = &host_logits_[d_.row_at(b, s)];
        const float *gp = &host_probabilities_[d_.row_at(b, s)];
        for (long long r = 0; r < V; ++r) l[static_cast<size_t>(r)] = gl[r];
        softmax_double(l.data(), V, p.data());
        long long best = 0;
        for (long long r = 0; r < V; ++r) {
          const double e = p[static_cast<size_t>(r)];
          if (!(std::fabs(gp[r] - e) <= 2e-5 * std::fabs(e) + 1e-12) && prob_errors[job]++ == 0 && report())
            std::fprintf(stderr, "%s: probability mismatch step %lld sequence %lld row %lld: expected %.9g, actual "
                         "%.9g\n", app, s, b, r, e, static_cast<double>(gp[r]));
          if (gp[r] > gp[best]) best = r;
        }
        if (host_generated_.get()[b * S + s] != best) {
          tok_errors[job] = 1;
          if (report())
            std::fprintf(stderr, "%s: token step %lld sequence %lld is %d, the first largest probability is at "
                         "%lld\n", app, s, b, host_generated_.get()[b * S + s], best);
        }
      }
    });
    long long probability_errors = 0, token_errors = 0;
    for (size_t j = 0; j < prob_errors.size(); ++j) probability_errors += prob_errors[j], token_errors += tok_errors[j];

    bool pass = normalized_errors == 0 && token_range_errors == 0 && activations_ok && weights_match_ &&
                total_logit_errors == 0 && probability_errors == 0 && token_errors == 0;
    std::fprintf(stderr,
                 "%s: implementation check %s: normalized %lld mismatches, %lld tokens out of range; converted "
                 "weights %s, activations %s; logits %lld mismatches over %lld sequences x %lld steps (worst "
                 "|error| / sum|terms| %.3g, bound %.3g); probabilities %lld mismatches; tokens %lld not the first "
                 "largest probability\n",
                 app, pass ? "PASS" : "FAIL", normalized_errors, token_range_errors, weights_match_ ? "exact" : "MISMATCH",
                 activations_ok ? "exact" : "MISMATCH", total_logit_errors, count, S, worst_logit, gamma,
                 probability_errors, token_errors);
    if (contract_) {
      // The control must also pass the production contract check unchanged.
      const bool production = l2c_decoder::verify(d_, *contract_, {host_generated_.get(), host_normalized_.data(),
                                                                   host_logits_.data(), host_probabilities_.data()});
      pass = pass && production;
    }
    return pass;
  }

  int c_;
  l2c_decoder::Dims d_;
  int fixture_;
  int fault_;
  float alpha_host_ = 1.0f;
  DeviceArray<float> embedding_, classifier_, norm_weight_, normalized_, logits_, probabilities_, partials_, alpha_;
  DeviceArray<int> prompts_, tokens_, generated_;
  PinnedArray<int> host_prompts_, host_generated_;
  std::vector<float> host_embedding_, host_classifier_;
  Operand weights_;
  std::vector<Operand> activations_;
  const float *other_decode_override_ = nullptr;
  std::vector<float> dequantized_weights_;
  float weight_decode_ = 1.0f;
  bool weights_match_ = true;
  std::unique_ptr<l2c_decoder::Expectation> contract_;
  std::vector<float> host_normalized_, host_logits_, host_probabilities_;
  std::vector<std::vector<uint8_t>> host_activation_bytes_;
};

// Dimensions with the decoder contract's limits and the experiment's alignment
// (decoder_lowprec.cu:1106-1127; scripts match the messages).
std::unique_ptr<LowprecWorkload> make_lowprec(int c, long long batch, long long width, long long vocab, long long steps,
                                              long long fixture, long long fault = 0) {
  using appproto::abort_run;
  using appproto::kUsage;
  if (fixture < 0 || fixture > 3) abort_run(kUsage, "fixture must be 0 (primary model) or 1, 2, 3 (got %lld)", fixture);
  if (batch < 1 || batch > (1LL << 20)) abort_run(kUsage, "batch must be in [1, 1048576] (got %lld)", batch);
  if (width < 2 || width > (1LL << 24) - 16) abort_run(kUsage, "width must be in [2, 16777200] (got %lld)", width);
  if (vocab < 2 || vocab > width)
    abort_run(kUsage, "vocab must satisfy 2 <= vocab <= width (got %lld, %lld)", vocab, width);
  if (steps < 2 || steps > 1024) abort_run(kUsage, "steps must be in [2, 1024] (got %lld)", steps);
  const long long max_fault = c == kNvfp4 ? 3 : c == kMxfp6 ? 2 : c == kBf16 ? 1 : 0;
  if (fault < 0 || fault > max_fault)
    abort_run(kUsage, "fault must be in [0, %lld] for case %s (got %lld)", max_fault, case_name(c), fault);
  if (c != kFp32 && (width % 128 != 0 || vocab % 4 != 0))
    abort_run(kUsage, "low precision cases need width %% 128 == 0 and vocab %% 4 == 0 (got width %lld, vocab %lld)",
         width, vocab);
  const double gib = static_cast<double>(1LL << 30);
  const double device = 4.0 * (2.0 * static_cast<double>(vocab) * width) +
                        4.0 * static_cast<double>(steps) * batch * (static_cast<double>(width) + 2.0 * vocab) +
                        2.0 * (static_cast<double>(vocab) + steps * static_cast<double>(batch)) * width;
  if (device > kDeviceLimitGiB * gib)
    abort_run(kUsage, "dimensions need %.1f GiB of device memory (limit %.0f)", device / gib, kDeviceLimitGiB);
  return std::make_unique<LowprecWorkload>(c, batch, width, vocab, steps, static_cast<int>(fixture),
                                           static_cast<int>(fault));
}

int g_case = kFp32;

std::unique_ptr<appproto::Application> make_workload(const std::string &preset, appproto::Settings &settings,
                                                     appproto::Assets &) {
  const long long fixture = settings.integer("fixture", 0);
  const bool dense = fixture != 0;
  const long long batch = settings.integer("batch", dense ? kFixtureBatch : kLargeBatch);
  const long long width = settings.integer("width", dense ? kFixtureWidth : kLargeWidth);
  const long long vocab = settings.integer("vocab", dense ? kFixtureVocab : kLargeVocab);
  const long long steps = settings.integer("steps", kLargeSteps);
  const long long fault = settings.integer("fault", 0);
  if (preset != "large") return nullptr;
  return make_lowprec(g_case, batch, width, vocab, steps, fixture, fault);
}

// ---------------------------------------------------------------------------
// --selftest: crafted rows through the device conversion against the host
// reference (element and scale ties, saturation, zero, tiny and subnormal
// blocks; 130 rows).
std::vector<float> crafted(long long rows, long long width) {
  std::vector<float> m(static_cast<size_t>(rows * width), 0.0f);
  auto at = [&](long long r, long long k) -> float & { return m[static_cast<size_t>(r * width + k)]; };
  at(0, 0) = 2688.0f;  // the tensor maximum: NVFP4 encode scale 1
  const float e2[16] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.0f, 5.5f,
                        -0.25f, -0.75f, -2.5f, -5.5f, 0.26f, -0.2f, 6.0f, 6.2f};
  const float e3[16] = {0.03125f, 0.09375f, 0.15625f, 0.21875f, 1.125f, 1.375f, 2.75f, 26.0f,
                        30.0f, -0.03125f, -0.09375f, -26.0f, 0.0f, 16.0f, 18.0f, 22.0f};
  for (int i = 0; i < 16; ++i) {
    at(1, i) = e2[i];
    at(1, 16 + i) = e2[i] * 0.75f;
    at(2, i) = e3[i];
    at(2, 32 + i) = e3[i] / 4.0f;
    at(2, 48 + i) = e3[i] / 4.0f;
  }
  const float sat[4] = {31.9f, 31.0f, 29.9f, 28.1f};
  for (int i = 0; i < 16; ++i) at(2, 16 + i) = i < 4 ? sat[i] : 1.0f;
  for (long long blk = 0; blk < std::min<long long>(8, width / 32); ++blk) {
    const float top = static_cast<float>((2.0 - std::ldexp(1.0, -static_cast<int>(blk) - 2)) * std::ldexp(1.0, static_cast<int>(blk) - 4));
    at(3, 32 * blk) = top;
    for (int i = 1; i < 32; ++i) at(3, 32 * blk + i) = top * (-0.99f + 1.97f * static_cast<float>(i - 1) / 30.0f);
  }
  for (int i = 0; i < 16; ++i) {
    at(4, i) = 1e-6f * static_cast<float>(i - 8);
    at(4, 16 + i) = 0.004f * static_cast<float>(i - 8);
  }
  for (int i = 0; i < 32; ++i) {
    at(4, 32 + i) = 1e-30f * static_cast<float>(i + 1);
    at(4, 64 + i) = 1e-40f * static_cast<float>(i - 15);
    at(4, 96 + i) = std::ldexp(1.0f, -126) * static_cast<float>(i);
  }
  for (long long i = 0; i < width / 16; ++i) {
    at(5, 16 * i) = 6.0f * (1.0f + 0.0625f * static_cast<float>(i % 16));
    at(5, 16 * i + 1) = -3.0f;
  }
  for (int i = 0; i < 32; ++i) {
    at(6, 32 + i) = -0.0f;
    at(6, 64 + i) = 0.5f;
  }
  uint64_t state = 7;
  for (long long r = 7; r < rows; ++r)
    for (long long k = 0; k < width; ++k) {
      state = state * 6364136223846793005ull + 1442695040888963407ull;
      const double u = static_cast<double>(state >> 11) * 0x1p-53;
      at(r, k) = static_cast<float>((u - 0.5) * std::ldexp(1.0, static_cast<int>(r % 12) - 8));
    }
  return m;
}

int run_selftest(int c) {
  const long long rows = 130, width = 256;
  auto workload = make_lowprec(c, rows, width, 128, 2, 0);
  hipStream_t stream;
  APP_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  workload->prepare(stream);
  const bool pass = workload->selftest(crafted(rows, width), rows);
  (void)hipStreamDestroy(stream);
  std::printf("%s: %s quantizer self-test\n", pass ? "PASS" : "FAIL", case_name(c));
  return pass ? appproto::kPass : appproto::kMismatch;
}

// ---------------------------------------------------------------------------
// --accuracy (spec.json "accuracy"): the primary model and the three fixtures.
appproto::Json metrics_json(const ErrorMetrics &m) {
  using appproto::Json;
  Json j = Json::object();
  j.add("rows", Json::whole(m.rows))
      .add("max_abs_error", Json::real(m.max_abs_error))
      .add("normalized_rms_error", Json::real(m.normalized_rms_error))
      .add("max_abs_probability_error", Json::real(m.max_abs_probability_error))
      .add("mean_total_variation", Json::real(m.mean_total_variation))
      .add("top1_agree", Json::whole(m.top1_agree));
  return j;
}

appproto::Json accuracy_dataset(int c, int fixture, hipStream_t stream, double *weight_ms) {
  using appproto::Json;
  auto w = fixture == 0 ? make_lowprec(c, kLargeBatch, kLargeWidth, kLargeVocab, kLargeSteps, 0)
                        : make_lowprec(c, kFixtureBatch, kFixtureWidth, kFixtureVocab, kLargeSteps, fixture);
  LowprecWorkload &d = *w;
  d.prepare(stream);
  APP_HIP(hipStreamSynchronize(stream));
  const long long B = d.batch(), W = d.width(), V = d.vocab(), S = d.steps();
  if (weight_ms) {
    std::vector<double> times;
    hipEvent_t start, stop;
    APP_HIP(hipEventCreate(&start));
    APP_HIP(hipEventCreate(&stop));
    for (int i = 0; i < 5; ++i) {
      APP_HIP(hipEventRecord(start, stream));
      d.convert_weights(stream);
      APP_HIP(hipEventRecord(stop, stream));
      APP_HIP(hipEventSynchronize(stop));
      float ms = 0.0f;
      APP_HIP(hipEventElapsedTime(&ms, start, stop));
      times.push_back(ms);
    }
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
    std::sort(times.begin(), times.end());
    *weight_ms = times[2];
  }
  // Fixed FP32 reference activations: step-0 rows, rmsnorm in float on the host.
  std::vector<float> row(static_cast<size_t>(W)), activations(static_cast<size_t>(B * W));
  auto embedding = [&](long long token) -> const float * {
    if (fixture != 0) return &d.host_embedding()[static_cast<size_t>(token * W)];
    std::fill(row.begin(), row.end(), 1.0f);
    row[static_cast<size_t>(token)] = 4.0f;
    return row.data();
  };
  for (long long b = 0; b < B; ++b) rmsnorm_float(embedding(b % V), W, &activations[static_cast<size_t>(b * W)]);
  APP_HIP(hipMemcpyAsync(d.normalized(0), activations.data(), activations.size() * 4, hipMemcpyHostToDevice, stream));
  d.enqueue_classifier(0, stream);
  APP_HIP(hipStreamSynchronize(stream));
  std::vector<float> logits(static_cast<size_t>(B * V));
  APP_HIP(hipMemcpy(logits.data(), d.logits(0), logits.size() * 4, hipMemcpyDeviceToHost));
  std::vector<double> reference(static_cast<size_t>(B * V)), actual(logits.begin(), logits.end());
  l2c_host::parallel_ranges(static_cast<size_t>(B), threads(), [&](size_t b0, size_t b1, size_t) {
    for (long long b = static_cast<long long>(b0); b < static_cast<long long>(b1); ++b) {
      const float *x = &activations[static_cast<size_t>(b * W)];
      for (long long r = 0; r < V; ++r) {
        double sum = 0.0;
        if (fixture == 0) {
          sum = x[(r + V - 1) % V];  // the one nonzero weight, 1.0
        } else {
          const float *wr = &d.host_classifier()[static_cast<size_t>(r * W)];
          for (long long k = 0; k < W; ++k) sum += static_cast<double>(x[k]) * wr[k];
        }
        reference[static_cast<size_t>(b * V + r)] = sum;
      }
    }
  });
  const ErrorMetrics classifier = compare_logits(reference, actual, B, V);

  // A complete decode (one application-scope invocation).
  d.scramble_outputs(stream);
  d.enqueue(appproto::Scope::kApplication, stream);
  APP_HIP(hipStreamSynchronize(stream));
  std::vector<int> expected(static_cast<size_t>(B * S));
  if (fixture == 0) {
    for (long long b = 0; b < B; ++b)
      for (long long s = 0; s < S; ++s) expected[static_cast<size_t>(b * S + s)] = static_cast<int>((b % V + s + 1) % V);
  } else {
    l2c_host::parallel_ranges(static_cast<size_t>(B), threads(), [&](size_t b0, size_t b1, size_t) {
      std::vector<double> o(static_cast<size_t>(W)), l(static_cast<size_t>(V));
      for (long long b = static_cast<long long>(b0); b < static_cast<long long>(b1); ++b) {
        long long token = b % V;
        for (long long s = 0; s < S; ++s) {
          rmsnorm_double(&d.host_embedding()[static_cast<size_t>(token * W)], W, o.data());
          for (long long r = 0; r < V; ++r) {
            const float *wr = &d.host_classifier()[static_cast<size_t>(r * W)];
            double sum = 0.0;
            for (long long k = 0; k < W; ++k) sum += o[static_cast<size_t>(k)] * wr[k];
            l[static_cast<size_t>(r)] = sum;
          }
          token = argmax_first(l.data(), V);
          expected[static_cast<size_t>(b * S + s)] = static_cast<int>(token);
        }
      }
    });
  }
  long long agree = 0;
  Json per_step = Json::list();
  for (long long s = 0; s < S; ++s) {
    long long n = 0;
    for (long long b = 0; b < B; ++b) n += d.generated()[b * S + s] == expected[static_cast<size_t>(b * S + s)];
    agree += n;
    per_step.push(Json::whole(n));
  }
  Json tokens = Json::object();
  tokens.add("agree", Json::whole(agree))
      .add("total", Json::whole(B * S))
      .add("per_step_agree", std::move(per_step))
      .add("reference", Json::text(fixture == 0 ? "analytic progression" : "double host decode"));
  Json out = Json::object();
  out.add("dataset", Json::text(fixture == 0 ? "primary" : "fixture" + std::to_string(fixture)))
      .add("batch", Json::whole(B))
      .add("width", Json::whole(W))
      .add("vocab", Json::whole(V))
      .add("steps", Json::whole(S))
      .add("classifier_error", metrics_json(classifier))
      .add("tokens", std::move(tokens));
  if (fixture == 0) {
    const l2c_decoder::Dims dims{B, W, V, S};
    const l2c_decoder::Expectation production(dims);
    std::vector<float> o(dims.activation_count()), l(dims.row_count()), p(dims.row_count());
    d.download_outputs(o.data(), l.data(), p.data());
    std::fprintf(stderr, "%s: production FP32 tolerance check of the %s decode (reported, not required):\n",
                 appproto::program(), case_name(c));
    const bool pass = l2c_decoder::verify(dims, production, {d.generated(), o.data(), l.data(), p.data()});
    out.add("production_fp32_tolerance_pass", Json::flag(pass));
  }
  std::fprintf(stderr, "%s: accuracy %s fixture %d: max |error| %.3g, normalized RMS %.3g, max |probability error| "
               "%.3g, tokens %lld/%lld\n", appproto::program(), case_name(c), fixture, classifier.max_abs_error,
               classifier.normalized_rms_error, classifier.max_abs_probability_error, agree, B * S);
  return out;
}

int run_accuracy(int c, int argc, const char *const *argv, std::string *record, bool print) {
  std::string json_out;
  for (int i = 1; i < argc; ++i) {
    const std::string flag = argv[i];
    if (flag == "--accuracy") continue;
    if (flag == "--json-out" && i + 1 < argc) json_out = argv[++i];
    else appproto::abort_run(appproto::kUsage, "--accuracy takes only --json-out PATH (got %s)", flag.c_str());
  }
  hipStream_t stream;
  APP_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  double weight_ms = 0.0;
  appproto::Json datasets = appproto::Json::list();
  for (int fixture = 0; fixture <= 3; ++fixture)
    datasets.push(accuracy_dataset(c, fixture, stream, fixture == 0 ? &weight_ms : nullptr));
  (void)hipStreamDestroy(stream);
  hipDeviceProp_t prop{};
  int device = 0;
  APP_HIP(hipGetDevice(&device));
  APP_HIP(hipGetDeviceProperties(&prop, device));
  using appproto::Json;
  Json result = Json::object();
  result.add("schema", Json::text("blackwell_experiments.lowprec_accuracy/1"))
      .add("identity", Json::text(std::string("blackwell-experiments/lowprec-decoder-classifier/") + case_name(c)))
      .add("case", Json::text(case_name(c)))
      .add("spec_sha256", Json::text(kSpecSha256))
      .add("device", Json::text(prop.name))
      .add("weight_conversion_ms_median_of_5", Json::real(weight_ms))
      .add("datasets", std::move(datasets))
      .add("status", Json::text("accuracy"));
  const std::string line = result.dump();
  if (record) *record = line;
  if (print) std::printf("RESULT %s\n", line.c_str());
  if (!json_out.empty()) {
    FILE *file = std::fopen(json_out.c_str(), "w");
    if (!file || std::fprintf(file, "%s\n", line.c_str()) < 0 || std::fclose(file))
      appproto::abort_run(appproto::kUsage, "cannot write %s", json_out.c_str());
  }
  return appproto::kPass;
}

const appproto::Provenance kBuild{"gfx950", kSpecSha256, "v1", "4a75f8d743ef7fe755822bab0ea0fb78009c145b"};
const char kProgram[] = "decoder_lowprec";

// The modes of decoder_lowprec.cu:1414-1420: --accuracy, --selftest, else the
// loom_private protocol.
int dispatch(int c, int argc, const char *const *argv, std::string *record, bool print) {
  if (c < kFp32 || c > kNvfp4) {
    std::fprintf(stderr, "lowprec: case must be 0 (fp32), 1 (bf16), 2 (mxfp6) or 3 (nvfp4) (got %d)\n", c);
    return appproto::kUsage;
  }
  appproto::set_program(kProgram);
  g_case = c;
  try {
    for (int i = 1; i < argc; ++i) {
      if (std::string(argv[i]) == "--accuracy") return run_accuracy(c, argc, argv, record, print);
      if (std::string(argv[i]) == "--selftest") return run_selftest(c);
    }
  } catch (const appproto::Abort &a) {
    std::fprintf(stderr, "%s: %s\n", appproto::program(), a.what());
    return a.code();
  }
  return appproto::run_protocol(kProgram, argc, argv, make_workload, kBuild, record, print);
}

}  // namespace

extern "C" int l2c_lowprec_main(int lowprec_case, int argc, const char *const *argv, char *record, size_t capacity) {
  std::string text;
  const int code = dispatch(lowprec_case, argc, argv, &text, false);
  if (record != nullptr && capacity > 0) {
    std::strncpy(record, text.c_str(), capacity - 1);
    record[capacity - 1] = '\0';
  }
  return code;
}

extern "C" int l2c_lowprec_run(int lowprec_case, int argc, const char *const *argv) {
  return dispatch(lowprec_case, argc, argv, nullptr, true);
}

extern "C" int l2c_lowprec_host_quantize(int lowprec_case, const float *x, int rows, int width, uint16_t *codes,
                                         uint8_t *scales, float *decode) {
  if (lowprec_case < kBf16 || lowprec_case > kNvfp4 || rows < 0 || width <= 0 || !x || !codes) return 2;
  const long long block = lowprec_case == kMxfp6 ? 32 : 16;
  if (lowprec_case != kBf16 && (width % block != 0 || !scales)) return 2;
  const Quantized q = quantize(lowprec_case, x, rows, width);
  std::copy(q.codes.begin(), q.codes.end(), codes);
  if (lowprec_case != kBf16) std::copy(q.scales.begin(), q.scales.end(), scales);
  if (decode) *decode = q.decode;
  return 0;
}

extern "C" int l2c_lowprec_fixture(int seed, int width, int vocab, float *embedding, float *classifier) {
  if (width <= 0 || vocab <= 0 || !embedding || !classifier) return 2;
  lowprec::fixture(seed, width, vocab, embedding, classifier);
  return 0;
}

extern "C" int l2c_lowprec_crafted(int rows, int width, float *out) {
  if (rows < 7 || width < 128 || width % 32 != 0 || !out) return 2;
  const std::vector<float> m = crafted(rows, width);
  std::copy(m.begin(), m.end(), out);
  return 0;
}
