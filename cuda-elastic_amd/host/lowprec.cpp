// The lowprec classifier experiment on MI355X (experiments/blackwell/lowprec):
// the llama2c decoder of loom-private/llama2c-decoder with only its dense
// classifier replaced, case by case, by a BF16, MXFP6 or NVFP4 contraction, or
// kept in FP32 (the control). Three modes:
//   the loom_private protocol   check / bench / profile (app_protocol.h)
//   --selftest                  the device conversion of a crafted matrix
//                               against the host quantizer
//   --accuracy                  numerical quality on the primary model and
//                               the three dense fixtures
//
// Parts of this file:
//   HostModel             what the host knows of the model the GPU runs
//   ClassifierExperiment  the application: device state, the per-step
//                         enqueue, and host snapshots of an invocation
//   Stage, Audit          the implementation check, one stage at a time
//   Assessment            one dataset of --accuracy
// Formats and their device planes are in lowprec_formats.h; the host
// quantizer, fixtures and double references in lowprec_reference.h.
//
// What callers rely on (option names, exit codes, the record schemas and
// scope strings, the dimension messages) follows spec.json and the
// reference's tests/run_tests.sh; the organisation is this build's own.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <numeric>
#include <string>
#include <thread>
#include <vector>

#include "../../include/l2c.h"
#include "../../include/l2c_harness.h"
#include "app_protocol.h"
#include "decoder_contract.h"
#include "lowprec_formats.h"
#include "lowprec_reference.h"
#include "parallel.h"

namespace {

// L2C_LOWPREC_AMAX_IN_RMSNORM=1: a step's rmsnorm also takes the activation
// maximum that NVFP4's tensor scale needs (l2c_decoder_rmsnorm_absmax), in place
// of the format's own pass over the activations. Read once.
bool amax_in_rmsnorm() {
  static const bool on = [] {
    const char *v = std::getenv("L2C_LOWPREC_AMAX_IN_RMSNORM");
    return v && std::strcmp(v, "1") == 0;
  }();
  return on;
}

using appproto::Json;
using l2c_decoder::DeviceArray;
using l2c_decoder::device_array;
using l2c_decoder::Dims;
using l2c_decoder::PinnedArray;
using l2c_decoder::pinned_array;
using namespace lowprec;

// The experiment's two shapes (spec.json "dimensions").
constexpr Dims kPrimary{1024, 16384, 8192, 4};
constexpr Dims kFixtureShape{64, 1024, 128, 4};
constexpr double kDeviceLimitGiB = 64.0;
// sha256 of experiments/blackwell/lowprec/spec.json, recorded in every result.
constexpr const char *kSpecSha256 = "1a56ed12366829cbf1b952d99267143f4d74f64411858cb6e7748e389616a64c";
constexpr const char kProgram[] = "decoder_lowprec";
// Failures printed per check stage before the rest are only counted.
constexpr long long kShownPerStage = 5;

int host_threads() {
  return static_cast<int>(std::max(1u, std::min(16u, std::thread::hardware_concurrency())));
}

// f(i) for i in [0, n) over the host threads, in contiguous ranges.
template <typename F>
void spread(long long n, F f) {
  l2c_host::parallel_ranges(static_cast<size_t>(n), host_threads(), [&](size_t i0, size_t i1, size_t) {
    for (size_t i = i0; i < i1; ++i) f(static_cast<long long>(i));
  });
}

std::string identity(int c) { return std::string("blackwell-experiments/lowprec-decoder-classifier/") + case_name(c); }

// ---------------------------------------------------------------------------
// HostModel: the primary (synthetic) model or a dense fixture, as the host
// evaluates it. The synthetic model is never materialized on the host except
// where a caller asks for the whole classifier.

class HostModel {
 public:
  static HostModel synthetic(long long width, long long vocab) { return HostModel(0, width, vocab); }
  static HostModel dense(int seed, long long width, long long vocab) {
    HostModel m(seed, width, vocab);
    const size_t n = static_cast<size_t>(width * vocab);
    m.embedding_.resize(n);
    m.classifier_.resize(n);
    fixture(seed, width, vocab, m.embedding_.data(), m.classifier_.data());
    return m;
  }

  int seed() const { return seed_; }
  bool is_synthetic() const { return seed_ == 0; }
  long long width() const { return width_; }
  long long vocab() const { return vocab_; }
  long long prompt(long long sequence) const { return sequence % vocab_; }

  // Embedding row of a token; the synthetic row (1, and 4 at the token's own
  // column) is written into *scratch.
  const float *embedding_row(long long token, std::vector<float> *scratch) const {
    if (!is_synthetic()) return &embedding_[static_cast<size_t>(token * width_)];
    scratch->assign(static_cast<size_t>(width_), 1.0f);
    (*scratch)[static_cast<size_t>(token)] = 4.0f;
    return scratch->data();
  }

  // The classifier's only nonzero column in row r of the synthetic model.
  long long synthetic_column(long long r) const { return (r + vocab_ - 1) % vocab_; }

  // The whole classifier, [vocab][width] floats.
  std::vector<float> classifier() const {
    if (!is_synthetic()) return classifier_;
    std::vector<float> w(static_cast<size_t>(vocab_ * width_), 0.0f);
    for (long long r = 0; r < vocab_; ++r) w[static_cast<size_t>(r * width_ + synthetic_column(r))] = 1.0f;
    return w;
  }

  // Logit r of activations x: the double dot product with classifier row r.
  double logit(const float *x, long long r) const {
    if (is_synthetic()) return x[synthetic_column(r)];
    const float *w = &classifier_[static_cast<size_t>(r * width_)];
    double sum = 0.0;
    for (long long k = 0; k < width_; ++k) sum += static_cast<double>(x[k]) * w[k];
    return sum;
  }

  void upload(float *embedding, float *classifier, float *norm_weight, hipStream_t stream) const {
    if (is_synthetic()) {
      APP_L2C(l2c_decoder_init_model(embedding, classifier, norm_weight, static_cast<int>(width_),
                                     static_cast<int>(vocab_), stream));
      return;
    }
    const std::vector<float> ones(static_cast<size_t>(width_), 1.0f);
    APP_HIP(hipMemcpyAsync(embedding, embedding_.data(), embedding_.size() * 4, hipMemcpyHostToDevice, stream));
    APP_HIP(hipMemcpyAsync(classifier, classifier_.data(), classifier_.size() * 4, hipMemcpyHostToDevice, stream));
    APP_HIP(hipMemcpyAsync(norm_weight, ones.data(), ones.size() * 4, hipMemcpyHostToDevice, stream));
    APP_HIP(hipStreamSynchronize(stream));  // `ones` leaves scope
  }

  // Greedy tokens [batch][steps] in exact arithmetic: the synthetic model
  // moves every token to its successor; a dense model is decoded on the host
  // in double (rmsnorm, every logit, first largest).
  std::vector<int> reference_tokens(long long batch, long long steps) const {
    std::vector<int> out(static_cast<size_t>(batch * steps));
    spread(batch, [&](long long b) {
      std::vector<double> normalized(static_cast<size_t>(width_)), logits(static_cast<size_t>(vocab_));
      std::vector<float> scratch;
      long long token = prompt(b);
      for (long long s = 0; s < steps; ++s) {
        if (is_synthetic()) {
          token = (token + 1) % vocab_;
        } else {
          rmsnorm_double(embedding_row(token, &scratch), width_, normalized.data());
          for (long long r = 0; r < vocab_; ++r) {
            const float *w = &classifier_[static_cast<size_t>(r * width_)];
            double sum = 0.0;
            for (long long k = 0; k < width_; ++k) sum += normalized[static_cast<size_t>(k)] * w[k];
            logits[static_cast<size_t>(r)] = sum;
          }
          token = argmax_first(logits.data(), vocab_);
        }
        out[static_cast<size_t>(b * steps + s)] = static_cast<int>(token);
      }
    });
    return out;
  }

 private:
  HostModel(int seed, long long width, long long vocab) : seed_(seed), width_(width), vocab_(vocab) {}
  int seed_;
  long long width_, vocab_;
  std::vector<float> embedding_, classifier_;
};

// ---------------------------------------------------------------------------
// Host copy of what one invocation left on the device.

struct Snapshot {
  std::vector<int> generated;                           // [batch][steps]
  std::vector<float> normalized, logits, probabilities;  // [steps][batch][...]
  std::vector<PlaneBytes> activations;                   // per step, the format's planes
  std::vector<float> alpha;                              // NVFP4, per step
};

// The converted weights, compared once against the host quantizer.
struct WeightReading {
  long long values = 0, differing = 0;
  Quantized host;                // the host quantizer's codes of the FP32 weights
  std::vector<float> values_f;   // their values without the NVFP4 tensor scale
};

// ---------------------------------------------------------------------------
// Stage: one stage of the implementation check. Counts compared and failed
// items from any thread and prints the first few failures.

class Stage {
 public:
  explicit Stage(const char *name) : name_(name) {}
  const char *name() const { return name_; }
  void compared(long long n) { checked_ += n; }
  void failed(const char *format, ...) __attribute__((format(printf, 2, 3))) {
    if (failures_.fetch_add(1) >= kShownPerStage) return;
    char line[512];
    va_list args;
    va_start(args, format);
    std::vsnprintf(line, sizeof line, format, args);
    va_end(args);
    std::lock_guard<std::mutex> lock(print_);
    std::fprintf(stderr, "%s: %s: %s\n", appproto::program(), name_, line);
  }
  // A failure already reported elsewhere (counted, not printed).
  void failed_silently(long long n) { failures_ += n; }
  void worst(double ratio) {
    std::lock_guard<std::mutex> lock(print_);
    worst_ = std::max(worst_, ratio);
  }
  bool ok() const { return failures_.load() == 0; }
  long long failures() const { return failures_.load(); }
  std::string tally() const {
    char text[160];
    std::snprintf(text, sizeof text, "%s %lld/%lld failed", name_, failures_.load(), checked_.load());
    std::string out = text;
    if (worst_ > 0.0) {
      std::snprintf(text, sizeof text, " (largest passing error / bound %.3g)", worst_);
      out += text;
    }
    return out;
  }

 private:
  const char *name_;
  std::atomic<long long> checked_{0}, failures_{0};
  double worst_ = 0.0;
  std::mutex print_;
};

// Codes, scales and the NVFP4 decode scale of `device` against `host`, the
// same [rows][width] operand; the differences go to `stage`.
void match_codes(Stage &stage, const char *what, const Quantized &host, const Quantized &device, long long width) {
  stage.compared(static_cast<long long>(host.codes.size() + host.scales.size()));
  for (size_t i = 0; i < host.codes.size(); ++i)
    if (host.codes[i] != device.codes[i])
      stage.failed("%s code mismatch at row %lld column %lld: host quantizer 0x%x, device 0x%x", what,
                   static_cast<long long>(i) / width, static_cast<long long>(i) % width, host.codes[i],
                   device.codes[i]);
  const long long blocks_per_row = host.scales.empty() ? 1 : static_cast<long long>(host.scales.size()) /
                                                                 (static_cast<long long>(host.codes.size()) / width);
  for (size_t i = 0; i < host.scales.size(); ++i)
    if (host.scales[i] != device.scales[i])
      stage.failed("%s scale mismatch at row %lld block %lld: host quantizer 0x%02x, device 0x%02x", what,
                   static_cast<long long>(i) / blocks_per_row, static_cast<long long>(i) % blocks_per_row,
                   host.scales[i], device.scales[i]);
  if (!(host.decode == device.decode))
    stage.failed("%s tensor decode scale mismatch: host %.9g, device %.9g", what, static_cast<double>(host.decode),
                 static_cast<double>(device.decode));
}

// ---------------------------------------------------------------------------
// ClassifierExperiment: the decoder with the case's classifier, under the
// loom_private protocol. Per step on one stream: rmsnorm of the current
// tokens' embedding rows -> the case's activation conversion -> its
// contraction -> softmax + argmax, which writes the next tokens.

class ClassifierExperiment final : public appproto::Application {
 public:
  // Test hooks (--set fault=N, check only), planted in what the host reads
  // back rather than in the kernels: 1 moves one step-0 activation code one
  // step toward zero, 2 exchanges two differing neighbouring step-0 block
  // scales, 3 divides the logits by alpha (a contraction that dropped alpha).
  enum Fault { kNoFault = 0, kRounding = 1, kScaleLayout = 2, kAlpha = 3 };

  ClassifierExperiment(int lowprec_case, const Dims &dims, HostModel model, int fault)
      : case_(lowprec_case), d_(dims), model_(std::move(model)), fault_(fault), format_(make_format(lowprec_case)) {}

  appproto::AppInfo info() const override {
    appproto::AppInfo i;
    i.identity = identity(case_);
    i.dimensions.add("batch", Json::whole(d_.batch))
        .add("width", Json::whole(d_.width))
        .add("vocab", Json::whole(d_.vocab))
        .add("steps", Json::whole(d_.steps))
        .add("fixture", Json::whole(model_.seed()))
        .add("case", Json::text(case_name(case_)))
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

  const Dims &dims() const { return d_; }
  const HostModel &model() const { return model_; }
  int lowprec_case() const { return case_; }
  float *normalized(long long step) const { return normalized_.get() + d_.activation_at(0, step); }
  float *logits(long long step) const { return logits_.get() + d_.row_at(0, step); }
  double setup_encode_ms() const { return setup_encode_ms_; }

  void prepare(hipStream_t stream) override {
    const size_t model_values = static_cast<size_t>(d_.vocab * d_.width);
    embedding_ = device_array<float>(model_values);
    classifier_ = device_array<float>(model_values);
    norm_weight_ = device_array<float>(static_cast<size_t>(d_.width));
    prompts_ = device_array<int>(static_cast<size_t>(d_.batch));
    tokens_ = device_array<int>(static_cast<size_t>(d_.batch));
    generated_ = device_array<int>(d_.token_count());
    normalized_ = device_array<float>(d_.activation_count());
    logits_ = device_array<float>(d_.row_count());
    probabilities_ = device_array<float>(d_.row_count());
    pinned_prompts_ = pinned_array<int>(static_cast<size_t>(d_.batch));
    pinned_generated_ = pinned_array<int>(d_.token_count());
    for (long long b = 0; b < d_.batch; ++b) pinned_prompts_.get()[b] = static_cast<int>(model_.prompt(b));
    model_.upload(embedding_.get(), classifier_.get(), norm_weight_.get(), stream);
    weights_ = format_->allocate(d_.vocab, d_.width);
    for (long long s = 0; s < d_.steps; ++s) step_inputs_.push_back(format_->allocate(d_.batch, d_.width));
    if (case_ == kNvfp4) alpha_ = device_array<float>(static_cast<size_t>(d_.steps));
    setup_encode_ms_ = time_ms(stream, [&] { encode_weights(stream); });
    std::fprintf(stderr, "%s: %s classifier, %s model: weights converted in %.3f ms at setup\n", appproto::program(),
                 case_name(case_), model_.is_synthetic() ? "synthetic" : ("fixture " + std::to_string(model_.seed())).c_str(),
                 setup_encode_ms_);
  }

  void encode_weights(hipStream_t stream) { format_->encode(classifier_.get(), weights_, nullptr, nullptr, stream); }

  // Times `work` on `stream` with a pair of events, in milliseconds.
  template <typename F>
  static double time_ms(hipStream_t stream, F work) {
    hipEvent_t begin, end;
    APP_HIP(hipEventCreate(&begin));
    APP_HIP(hipEventCreate(&end));
    APP_HIP(hipEventRecord(begin, stream));
    work();
    APP_HIP(hipEventRecord(end, stream));
    APP_HIP(hipEventSynchronize(end));
    float ms = 0.0f;
    APP_HIP(hipEventElapsedTime(&ms, begin, end));
    (void)hipEventDestroy(begin);
    (void)hipEventDestroy(end);
    return ms;
  }

  void enqueue(appproto::Scope scope, hipStream_t stream) override {
    const bool application = scope == appproto::Scope::kApplication;
    const size_t token_bytes = static_cast<size_t>(d_.batch) * sizeof(int);
    if (application)
      APP_HIP(hipMemcpyAsync(prompts_.get(), pinned_prompts_.get(), token_bytes, hipMemcpyHostToDevice, stream));
    APP_HIP(hipMemcpyAsync(tokens_.get(), prompts_.get(), token_bytes, hipMemcpyDeviceToDevice, stream));
    const int B = static_cast<int>(d_.batch), W = static_cast<int>(d_.width), V = static_cast<int>(d_.vocab),
              S = static_cast<int>(d_.steps);
    // spec.json ("based_on.note") keeps the production rmsnorm unchanged in every
    // case, so a format's activation maximum comes from the rmsnorm only on
    // request (L2C_LOWPREC_AMAX_IN_RMSNORM=1); the rmsnorm's output is the same.
    unsigned *absmax = amax_in_rmsnorm() ? format_->activation_absmax() : nullptr;
    for (int s = 0; s < S; ++s) {
      if (absmax)
        APP_L2C(l2c_decoder_rmsnorm_absmax(normalized(s), tokens_.get(), embedding_.get(), norm_weight_.get(), W, V,
                                           B, absmax, stream));
      else
        APP_L2C(l2c_decoder_rmsnorm(normalized(s), tokens_.get(), embedding_.get(), norm_weight_.get(), W, V, B,
                                    stream));
      classify(s, stream, absmax != nullptr);
      APP_L2C(l2c_decoder_softmax_argmax(probabilities_.get() + d_.row_at(0, s), logits(s), tokens_.get(),
                                         generated_.get(), V, B, S, s, stream));
    }
    if (application)
      APP_HIP(hipMemcpyAsync(pinned_generated_.get(), generated_.get(), d_.token_count() * sizeof(int),
                             hipMemcpyDeviceToHost, stream));
  }

  // The case's classifier for one step: whatever normalized(step) holds is
  // converted (NVFP4: with that step's alpha) and contracted with the weights.
  // `after_rmsnorm`: the step's rmsnorm filled the format's activation maximum
  // (activation_absmax), so the encoding takes it instead of its own pass.
  void classify(long long step, hipStream_t stream, bool after_rmsnorm) {
    DeviceTensor &x = step_inputs_[static_cast<size_t>(step)];
    float *alpha = alpha_ ? alpha_.get() + step : nullptr;
    if (after_rmsnorm)
      format_->encode_activations(normalized(step), x, alpha, format_->decode_scale(weights_), stream);
    else
      format_->encode(normalized(step), x, alpha, format_->decode_scale(weights_), stream);
    format_->contract(logits(step), normalized(step), x, classifier_.get(), weights_, alpha,
                      static_cast<int>(d_.batch), static_cast<int>(d_.width), static_cast<int>(d_.vocab), stream);
  }

  void scramble_outputs(hipStream_t stream) override {
    const auto fill = [&](void *p, size_t bytes) { APP_HIP(hipMemsetAsync(p, 0xFF, bytes, stream)); };
    fill(prompts_.get(), static_cast<size_t>(d_.batch) * sizeof(int));
    fill(tokens_.get(), static_cast<size_t>(d_.batch) * sizeof(int));
    fill(generated_.get(), d_.token_count() * sizeof(int));
    fill(normalized_.get(), d_.activation_count() * sizeof(float));
    fill(logits_.get(), d_.row_count() * sizeof(float));
    fill(probabilities_.get(), d_.row_count() * sizeof(float));
    for (const DeviceTensor &x : step_inputs_) poison(x, stream);
    if (alpha_) fill(alpha_.get(), static_cast<size_t>(d_.steps) * sizeof(float));
    std::memset(pinned_generated_.get(), 0xFF, d_.token_count() * sizeof(int));
  }

  void derive_expected() override {
    APP_HIP(hipDeviceSynchronize());
    if (case_ != kFp32) read_weights();
    if (case_ == kFp32 && model_.is_synthetic()) production_ = std::make_unique<l2c_decoder::Expectation>(d_);
  }

  Snapshot snapshot() const {
    Snapshot s;
    s.generated.assign(pinned_generated_.get(), pinned_generated_.get() + d_.token_count());
    s.normalized.resize(d_.activation_count());
    s.logits.resize(d_.row_count());
    s.probabilities.resize(d_.row_count());
    APP_HIP(hipMemcpy(s.normalized.data(), normalized_.get(), s.normalized.size() * 4, hipMemcpyDeviceToHost));
    APP_HIP(hipMemcpy(s.logits.data(), logits_.get(), s.logits.size() * 4, hipMemcpyDeviceToHost));
    APP_HIP(hipMemcpy(s.probabilities.data(), probabilities_.get(), s.probabilities.size() * 4, hipMemcpyDeviceToHost));
    for (const DeviceTensor &x : step_inputs_) s.activations.push_back(download(x));
    if (alpha_) {
      s.alpha.resize(static_cast<size_t>(d_.steps));
      APP_HIP(hipMemcpy(s.alpha.data(), alpha_.get(), s.alpha.size() * 4, hipMemcpyDeviceToHost));
    }
    return s;
  }

  bool outputs_match() override;

  // The generated tokens as the last application-scope invocation downloaded
  // them, then whatever the last check read back (nothing outside a check).
  uint64_t outputs_digest() const override {
    appproto::Digest h;
    h.add(pinned_generated_.get(), d_.token_count() * sizeof(int))
        .add(last_.normalized.data(), last_.normalized.size() * 4)
        .add(last_.logits.data(), last_.logits.size() * 4)
        .add(last_.probabilities.data(), last_.probabilities.size() * 4)
        .add(last_.alpha.data(), last_.alpha.size() * 4);
    for (const PlaneBytes &planes : last_.activations)
      for (const std::vector<uint8_t> &p : planes) h.add(p.data(), p.size());
    return h.value();
  }

  const Format &format() const { return *format_; }
  const WeightReading &weight_reading() const { return weights_read_; }
  const l2c_decoder::Expectation *production() const { return production_.get(); }
  int fault() const { return fault_; }

 private:
  // The converted weights against the host quantizer of the FP32 weights,
  // once (they are not touched by invocations), and their host values for the
  // logit check.
  void read_weights() {
    const std::vector<float> w = model_.classifier();
    weights_read_.host = quantize(case_, w.data(), d_.vocab, d_.width);
    std::string defect;
    const Quantized device = format_->unpack(download(weights_), d_.vocab, d_.width, &defect);
    Stage stage("converted weights");
    match_codes(stage, "weights", weights_read_.host, device, d_.width);
    if (!defect.empty()) stage.failed("weights: %s", defect.c_str());
    weights_read_.values = static_cast<long long>(w.size());
    weights_read_.differing = stage.failures();
    weights_read_.values_f.resize(w.size());
    spread(d_.vocab, [&](long long r) {
      for (long long k = 0; k < d_.width; ++k)
        weights_read_.values_f[static_cast<size_t>(r * d_.width + k)] = dequantized(case_, weights_read_.host, d_.width, r, k);
    });
  }

  int case_;
  Dims d_;
  HostModel model_;
  int fault_;
  std::unique_ptr<Format> format_;
  DeviceArray<float> embedding_, classifier_, norm_weight_, normalized_, logits_, probabilities_, alpha_;
  DeviceArray<int> prompts_, tokens_, generated_;
  PinnedArray<int> pinned_prompts_, pinned_generated_;
  DeviceTensor weights_;
  std::vector<DeviceTensor> step_inputs_;
  double setup_encode_ms_ = 0.0;
  WeightReading weights_read_;
  std::unique_ptr<l2c_decoder::Expectation> production_;
  Snapshot last_;
};

// ---------------------------------------------------------------------------
// Audit: spec.json "implementation_check". Each stage compares one thing the
// GPU produced with a host computation from the GPU's own inputs to that
// stage, so an implementation passes whatever its precision.

class Audit {
 public:
  Audit(const ClassifierExperiment &app, const Snapshot &got) : app_(app), got_(got), d_(app.dims()) {}

  bool run() {
    Stage normalized("normalized rows"), weights("converted weights"), inputs("converted activations"),
        logits("logits"), probabilities("probabilities"), tokens("tokens");
    check_normalized(normalized);
    const WeightReading &w = app_.weight_reading();
    weights.compared(w.values);
    if (w.differing) weights.failed_silently(w.differing);  // printed when the weights were read
    const std::vector<std::vector<float>> inputs_f = check_inputs(inputs);
    check_logits(logits, inputs_f);
    check_distribution(probabilities, tokens);
    const Stage *stages[] = {&normalized, &weights, &inputs, &logits, &probabilities, &tokens};
    bool pass = true;
    std::string summary;
    for (const Stage *s : stages) {
      pass = pass && s->ok();
      summary += (summary.empty() ? "" : "; ") + s->tally();
    }
    std::fprintf(stderr, "%s: implementation check %s: %s\n", appproto::program(), pass ? "PASS" : "FAIL",
                 summary.c_str());
    if (const l2c_decoder::Expectation *want = app_.production()) {
      // The FP32 control also passes the decoder's own contract check.
      const bool production = l2c_decoder::verify(
          d_, *want, {got_.generated.data(), got_.normalized.data(), got_.logits.data(), got_.probabilities.data()});
      pass = pass && production;
    }
    return pass;
  }

 private:
  int token_fed(long long b, long long s) const {
    return s == 0 ? static_cast<int>(app_.model().prompt(b)) : got_.generated[static_cast<size_t>(b * d_.steps + s - 1)];
  }

  // Every (step, sequence) row against rmsnorm in double of the embedding row
  // of the token the GPU fed into that step.
  void check_normalized(Stage &stage) {
    stage.compared(d_.steps * d_.batch);
    spread(d_.steps * d_.batch, [&](long long job) {
      const long long s = job / d_.batch, b = job % d_.batch;
      const int token = token_fed(b, s);
      if (token < 0 || token >= d_.vocab) {
        stage.failed("step %lld sequence %lld was fed token %d, outside the vocabulary", s, b, token);
        return;
      }
      std::vector<double> want(static_cast<size_t>(d_.width));
      std::vector<float> scratch;
      rmsnorm_double(app_.model().embedding_row(token, &scratch), d_.width, want.data());
      const float *row = &got_.normalized[d_.activation_at(b, s)];
      for (long long k = 0; k < d_.width; ++k) {
        const double e = want[static_cast<size_t>(k)];
        if (!(std::fabs(row[k] - e) <= l2c_decoder::kActivationTolerance * std::fabs(e) + l2c_decoder::kToleranceFloor)) {
          stage.failed("normalized mismatch at step %lld sequence %lld column %lld: host %.9g, device %.9g", s, b, k, e,
                       static_cast<double>(row[k]));
          return;  // one report per row
        }
      }
    });
  }

  // Each step's converted activations, bit for bit, against the host
  // quantizer of that step's GPU-normalized rows, and NVFP4's alpha against
  // d(activations) * d(weights). Returns the host values of the activations
  // (without the NVFP4 tensor scale), the operands the logit check multiplies.
  std::vector<std::vector<float>> check_inputs(Stage &stage) {
    const int c = app_.lowprec_case();
    std::vector<std::vector<float>> values(static_cast<size_t>(d_.steps));
    if (c == kFp32) return values;
    for (long long s = 0; s < d_.steps; ++s) {
      const Quantized host = quantize(c, &got_.normalized[d_.activation_at(0, s)], d_.batch, d_.width);
      std::string defect;
      Quantized device = app_.format().unpack(got_.activations[static_cast<size_t>(s)], d_.batch, d_.width, &defect);
      if (s == 0) plant(device);
      char what[40];
      std::snprintf(what, sizeof what, "step %lld", s);
      match_codes(stage, what, host, device, d_.width);
      if (!defect.empty()) stage.failed("%s: %s", what, defect.c_str());
      if (c == kNvfp4) {
        const float want = host.decode * app_.weight_reading().host.decode;
        const float have = got_.alpha[static_cast<size_t>(s)];
        stage.compared(1);
        if (!(have == want)) stage.failed("%s alpha mismatch: host %.9g, device %.9g", what, static_cast<double>(want), static_cast<double>(have));
      }
      std::vector<float> &v = values[static_cast<size_t>(s)];
      v.resize(static_cast<size_t>(d_.batch * d_.width));
      spread(d_.batch, [&](long long b) {
        for (long long k = 0; k < d_.width; ++k) v[static_cast<size_t>(b * d_.width + k)] = dequantized(c, host, d_.width, b, k);
      });
    }
    return values;
  }

  void plant(Quantized &q) const {
    const int c = app_.lowprec_case();
    if (app_.fault() == ClassifierExperiment::kRounding) {
      const unsigned magnitude_mask = c == kBf16 ? 0x7fffu : c == kMxfp6 ? 0x1fu : 0x7u;
      auto it = std::find_if(q.codes.begin(), q.codes.end(), [&](uint16_t v) { return (v & magnitude_mask) > 1; });
      if (it != q.codes.end()) --*it;
    } else if (app_.fault() == ClassifierExperiment::kScaleLayout) {
      for (size_t i = 0; i + 1 < q.scales.size(); i += 2)
        if (q.scales[i] != q.scales[i + 1]) {
          std::swap(q.scales[i], q.scales[i + 1]);
          break;
        }
    }
  }

  // Logits of up to 8 sequences spread over the batch (first and last
  // included), every step and vocabulary row, against the double product of
  // the host values of both operands times alpha. The bound gamma_K *
  // sum|a_k w_k| * |alpha| + 2^-23 |expected| + 1e-30, gamma_K = K u / (1 - K u)
  // with u = 2^-23, holds for FP32 accumulation in any order.
  void check_logits(Stage &stage, const std::vector<std::vector<float>> &inputs_f) {
    const int c = app_.lowprec_case();
    const long long probes = std::min<long long>(8, d_.batch);
    const double u = 0x1p-23, K = static_cast<double>(d_.width), gamma = K * u / (1.0 - K * u);
    std::vector<float> fp32_weights;
    if (c == kFp32) fp32_weights = app_.model().classifier();
    const std::vector<float> &weights = c == kFp32 ? fp32_weights : app_.weight_reading().values_f;
    stage.compared(probes * d_.steps * d_.vocab);
    spread(probes * d_.steps, [&](long long job) {
      const long long i = job / d_.steps, s = job % d_.steps;
      const long long b = probes == 1 ? 0 : i * (d_.batch - 1) / (probes - 1);
      const float *a = c == kFp32 ? &got_.normalized[d_.activation_at(b, s)]
                                  : &inputs_f[static_cast<size_t>(s)][static_cast<size_t>(b * d_.width)];
      const double alpha = c == kNvfp4 ? static_cast<double>(got_.alpha[static_cast<size_t>(s)]) : 1.0;
      const float *have = &got_.logits[d_.row_at(b, s)];
      double worst = 0.0;
      for (long long r = 0; r < d_.vocab; ++r) {
        const float *w = &weights[static_cast<size_t>(r * d_.width)];
        double dot = 0.0, magnitude = 0.0;
        for (long long k = 0; k < d_.width; ++k) {
          const double term = static_cast<double>(a[k]) * w[k];
          dot += term;
          magnitude += std::fabs(term);
        }
        const double want = dot * alpha;
        const double bound = gamma * magnitude * std::fabs(alpha) + u * std::fabs(want) + 1e-30;
        const double error = std::fabs(static_cast<double>(have[r]) - want);
        if (error <= bound) {
          worst = std::max(worst, error / bound);
        } else {
          stage.failed("logit mismatch at step %lld sequence %lld row %lld: host %.9g, device %.9g, bound %.3g", s, b, r,
                       want, static_cast<double>(have[r]), bound);
        }
      }
      stage.worst(worst);
    });
  }

  // Every (step, sequence): the probabilities against softmax in double of
  // the GPU's own logits, and the token against the first largest
  // probability the GPU wrote.
  void check_distribution(Stage &probabilities, Stage &tokens) {
    probabilities.compared(d_.steps * d_.batch);
    tokens.compared(d_.steps * d_.batch);
    spread(d_.steps * d_.batch, [&](long long job) {
      const long long s = job / d_.batch, b = job % d_.batch;
      const float *logits = &got_.logits[d_.row_at(b, s)];
      const float *p = &got_.probabilities[d_.row_at(b, s)];
      std::vector<double> wide(logits, logits + d_.vocab), want(static_cast<size_t>(d_.vocab));
      softmax_double(wide.data(), d_.vocab, want.data());
      for (long long r = 0; r < d_.vocab; ++r) {
        const double e = want[static_cast<size_t>(r)];
        if (!(std::fabs(p[r] - e) <= l2c_decoder::kProbabilityTolerance * std::fabs(e) + l2c_decoder::kToleranceFloor)) {
          probabilities.failed("probability mismatch at step %lld sequence %lld row %lld: host %.9g, device %.9g", s, b,
                               r, e, static_cast<double>(p[r]));
          break;
        }
      }
      const long long first_largest = std::max_element(p, p + d_.vocab) - p;
      const int token = got_.generated[static_cast<size_t>(b * d_.steps + s)];
      if (token != first_largest)
        tokens.failed("token mismatch at step %lld sequence %lld: device %d, first largest probability at %lld", s, b,
                      token, first_largest);
    });
  }

  const ClassifierExperiment &app_;
  const Snapshot &got_;
  const Dims d_;
};

bool ClassifierExperiment::outputs_match() {
  last_ = snapshot();
  if (fault_ == kAlpha)
    for (long long s = 0; s < d_.steps; ++s)
      for (size_t i = d_.row_at(0, s); i < d_.row_at(0, s + 1); ++i) last_.logits[i] /= last_.alpha[static_cast<size_t>(s)];
  return Audit(*this, last_).run();
}

// ---------------------------------------------------------------------------
// Dimensions: the decoder contract's limits, the cases' alignment, and the
// device memory the run needs (decoder_lowprec.cu:1106-1127 for the limits;
// tests match the wording).

void require(bool holds, const char *format, ...) __attribute__((format(printf, 2, 3)));
void require(bool holds, const char *format, ...) {
  if (holds) return;
  char reason[256];
  va_list args;
  va_start(args, format);
  std::vsnprintf(reason, sizeof reason, format, args);
  va_end(args);
  throw appproto::Abort(appproto::kUsage, reason);
}

// Device bytes per value of one encoded operand.
double encoded_bytes_per_value(int c) {
  switch (c) {
    case kBf16: return 2.0;
    case kMxfp6: return 0.75 + 1.0 / 32.0;
    case kNvfp4: return 0.5 + 1.0 / 16.0 + 2.0;
    default: return 0.0;
  }
}

std::unique_ptr<ClassifierExperiment> build_experiment(int c, const Dims &d, long long fixture, long long fault) {
  require(fixture >= 0 && fixture <= 3, "fixture must be 0 (primary model) or 1, 2, 3 (got %lld)", fixture);
  require(d.batch >= 1 && d.batch <= (1LL << 20), "batch must be in [1, 1048576] (got %lld)", d.batch);
  require(d.width >= 2 && d.width <= (1LL << 24) - 16, "width must be in [2, 16777200] (got %lld)", d.width);
  require(d.vocab >= 2 && d.vocab <= d.width, "vocab must satisfy 2 <= vocab <= width (got %lld, %lld)", d.vocab,
          d.width);
  require(d.steps >= 2 && d.steps <= 1024, "steps must be in [2, 1024] (got %lld)", d.steps);
  const long long most = c == kNvfp4 ? 3 : c == kMxfp6 ? 2 : c == kBf16 ? 1 : 0;
  require(fault >= 0 && fault <= most, "fault must be in [0, %lld] for case %s (got %lld)", most, case_name(c), fault);
  require(c == kFp32 || (d.width % 128 == 0 && d.vocab % 4 == 0),
          "low precision cases need width %% 128 == 0 and vocab %% 4 == 0 (got width %lld, vocab %lld)", d.width,
          d.vocab);
  const double W = static_cast<double>(d.width), V = static_cast<double>(d.vocab), B = static_cast<double>(d.batch),
               S = static_cast<double>(d.steps);
  const double bytes = 4.0 * 2.0 * V * W + 4.0 * S * B * (W + 2.0 * V) + encoded_bytes_per_value(c) * (V + S * B) * W;
  const double gib = static_cast<double>(1LL << 30);
  require(bytes <= kDeviceLimitGiB * gib, "dimensions need %.1f GiB of device memory (limit %.0f)", bytes / gib,
          kDeviceLimitGiB);
  HostModel model = fixture == 0 ? HostModel::synthetic(d.width, d.vocab)
                                 : HostModel::dense(static_cast<int>(fixture), d.width, d.vocab);
  return std::make_unique<ClassifierExperiment>(c, d, std::move(model), static_cast<int>(fault));
}

int g_case = kFp32;

std::unique_ptr<appproto::Application> protocol_factory(const std::string &preset, appproto::Settings &settings,
                                                        appproto::Assets &) {
  const long long fixture = settings.integer("fixture", 0);
  const Dims &shape = fixture != 0 ? kFixtureShape : kPrimary;
  const Dims d{settings.integer("batch", shape.batch), settings.integer("width", shape.width),
               settings.integer("vocab", shape.vocab), settings.integer("steps", kPrimary.steps)};
  const long long fault = settings.integer("fault", 0);
  if (preset != "large") return nullptr;
  return build_experiment(g_case, d, fixture, fault);
}

// ---------------------------------------------------------------------------
// --selftest: a crafted matrix through the device conversion against the host
// quantizer: element and scale ties, saturation, zero, tiny and subnormal-
// scale blocks, 130 rows so the row padding of the tiled layouts is used.

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
  bool pass = true;
  if (c != kFp32) {
    const std::vector<float> m = crafted(rows, width);
    std::unique_ptr<Format> format = make_format(c);
    DeviceArray<float> x = device_array<float>(m.size()), partner = device_array<float>(1),
                       alpha = device_array<float>(1);
    const float partner_decode = 0.75f;  // stands in for the weights' decode scale
    APP_HIP(hipMemcpy(x.get(), m.data(), m.size() * 4, hipMemcpyHostToDevice));
    APP_HIP(hipMemcpy(partner.get(), &partner_decode, 4, hipMemcpyHostToDevice));
    DeviceTensor t = format->allocate(rows, width);
    format->encode(x.get(), t, alpha.get(), partner.get(), nullptr);
    APP_HIP(hipDeviceSynchronize());
    std::string defect;
    const Quantized device = format->unpack(download(t), rows, width, &defect);
    const Quantized host = quantize(c, m.data(), rows, width);
    Stage stage("self-test");
    match_codes(stage, "crafted matrix", host, device, width);
    if (!defect.empty()) stage.failed("%s", defect.c_str());
    if (c == kNvfp4) {
      float have = 0.0f;
      APP_HIP(hipMemcpy(&have, alpha.get(), 4, hipMemcpyDeviceToHost));
      const float want = host.decode * partner_decode;
      stage.compared(1);
      if (!(have == want)) stage.failed("alpha %.9g, host %.9g", static_cast<double>(have), static_cast<double>(want));
    }
    std::fprintf(stderr, "%s: %s\n", appproto::program(), stage.tally().c_str());
    pass = stage.ok();
  }
  std::printf("%s: %s quantizer self-test\n", pass ? "PASS" : "FAIL", case_name(c));
  return pass ? appproto::kPass : appproto::kMismatch;
}

// ---------------------------------------------------------------------------
// Assessment: one dataset of --accuracy (spec.json "accuracy").
//   classifier error  the case's classifier alone on fixed step-0 activations
//                     (rmsnorm of each prompt's embedding row on the host, in
//                     float with a sequential square sum) against double
//                     logits of those activations and the FP32 weights
//   token agreement   one complete decode against the model's exact tokens
//   production        the decoder's contract check of that decode (primary)

class Assessment {
 public:
  Assessment(int c, int fixture) : fixture_(fixture) {
    const Dims &shape = fixture == 0 ? kPrimary : kFixtureShape;
    app_ = build_experiment(c, shape, fixture, 0);
  }

  Json run(hipStream_t stream, double *weight_ms) {
    ClassifierExperiment &app = *app_;
    app.prepare(stream);
    APP_HIP(hipStreamSynchronize(stream));
    if (weight_ms) *weight_ms = median_weight_encode_ms(stream, 5);
    const ErrorMetrics error = classifier_error(stream);
    const Dims &d = app.dims();
    app.scramble_outputs(stream);
    app.enqueue(appproto::Scope::kApplication, stream);
    APP_HIP(hipStreamSynchronize(stream));
    const Snapshot got = app.snapshot();
    const std::vector<int> want = app.model().reference_tokens(d.batch, d.steps);
    Json per_step = Json::list();
    long long agree = 0;
    for (long long s = 0; s < d.steps; ++s) {
      long long n = 0;
      for (long long b = 0; b < d.batch; ++b) {
        const size_t at = static_cast<size_t>(b * d.steps + s);
        n += got.generated[at] == want[at];
      }
      per_step.push(Json::whole(n));
      agree += n;
    }
    Json tokens = Json::object();
    tokens.add("agree", Json::whole(agree))
        .add("total", Json::whole(d.batch * d.steps))
        .add("per_step_agree", std::move(per_step))
        .add("reference", Json::text(fixture_ == 0 ? "analytic progression" : "double host decode"));
    Json errors = Json::object();
    errors.add("rows", Json::whole(error.rows))
        .add("max_abs_error", Json::real(error.max_abs_error))
        .add("normalized_rms_error", Json::real(error.normalized_rms_error))
        .add("max_abs_probability_error", Json::real(error.max_abs_probability_error))
        .add("mean_total_variation", Json::real(error.mean_total_variation))
        .add("top1_agree", Json::whole(error.top1_agree));
    Json out = Json::object();
    out.add("dataset", Json::text(fixture_ == 0 ? "primary" : "fixture" + std::to_string(fixture_)))
        .add("batch", Json::whole(d.batch))
        .add("width", Json::whole(d.width))
        .add("vocab", Json::whole(d.vocab))
        .add("steps", Json::whole(d.steps))
        .add("classifier_error", std::move(errors))
        .add("tokens", std::move(tokens));
    if (fixture_ == 0) {
      std::fprintf(stderr, "%s: the decoder's FP32 contract check of the %s decode follows (a precision result, "
                   "not required to pass):\n", appproto::program(), case_name(app.lowprec_case()));
      const l2c_decoder::Expectation contract(d);
      const bool pass = l2c_decoder::verify(
          d, contract, {got.generated.data(), got.normalized.data(), got.logits.data(), got.probabilities.data()});
      out.add("production_fp32_tolerance_pass", Json::flag(pass));
    }
    std::fprintf(stderr, "%s: accuracy of %s on %s: classifier max |error| %.3g, normalized RMS error %.3g, max "
                 "|probability error| %.3g; %lld of %lld tokens agree\n", appproto::program(),
                 case_name(app.lowprec_case()), fixture_ == 0 ? "the primary model" : ("fixture " + std::to_string(fixture_)).c_str(),
                 error.max_abs_error, error.normalized_rms_error, error.max_abs_probability_error, agree,
                 d.batch * d.steps);
    return out;
  }

 private:
  double median_weight_encode_ms(hipStream_t stream, int repetitions) {
    std::vector<double> ms;
    for (int i = 0; i < repetitions; ++i)
      ms.push_back(ClassifierExperiment::time_ms(stream, [&] { app_->encode_weights(stream); }));
    std::nth_element(ms.begin(), ms.begin() + repetitions / 2, ms.end());
    return ms[static_cast<size_t>(repetitions / 2)];
  }

  ErrorMetrics classifier_error(hipStream_t stream) {
    ClassifierExperiment &app = *app_;
    const Dims &d = app.dims();
    const HostModel &model = app.model();
    std::vector<float> x(static_cast<size_t>(d.batch * d.width));
    spread(d.batch, [&](long long b) {
      std::vector<float> scratch;
      rmsnorm_float(model.embedding_row(model.prompt(b), &scratch), d.width, &x[static_cast<size_t>(b * d.width)]);
    });
    APP_HIP(hipMemcpyAsync(app.normalized(0), x.data(), x.size() * 4, hipMemcpyHostToDevice, stream));
    app.classify(0, stream, false);  // normalized(0) comes from the host here
    std::vector<float> device(static_cast<size_t>(d.batch * d.vocab));
    APP_HIP(hipMemcpyAsync(device.data(), app.logits(0), device.size() * 4, hipMemcpyDeviceToHost, stream));
    APP_HIP(hipStreamSynchronize(stream));
    std::vector<double> reference(device.size()), actual(device.begin(), device.end());
    spread(d.batch, [&](long long b) {
      for (long long r = 0; r < d.vocab; ++r)
        reference[static_cast<size_t>(b * d.vocab + r)] = model.logit(&x[static_cast<size_t>(b * d.width)], r);
    });
    return compare_logits(reference, actual, d.batch, d.vocab);
  }

  int fixture_;
  std::unique_ptr<ClassifierExperiment> app_;
};

int run_accuracy(int c, int argc, const char *const *argv, std::string *record, bool print) {
  std::string json_out;
  for (int i = 1; i < argc; ++i) {
    const std::string arg = argv[i];
    if (arg == "--accuracy") continue;
    if (arg == "--json-out" && i + 1 < argc) {
      json_out = argv[++i];
      continue;
    }
    appproto::abort_run(appproto::kUsage, "--accuracy takes only --json-out PATH (got %s)", arg.c_str());
  }
  hipStream_t stream;
  APP_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  double weight_ms = 0.0;
  Json datasets = Json::list();
  for (int fixture = 0; fixture <= 3; ++fixture)
    datasets.push(Assessment(c, fixture).run(stream, fixture == 0 ? &weight_ms : nullptr));
  (void)hipStreamDestroy(stream);
  int device = 0;
  hipDeviceProp_t props{};
  APP_HIP(hipGetDevice(&device));
  APP_HIP(hipGetDeviceProperties(&props, device));
  Json result = Json::object();
  result.add("schema", Json::text("blackwell_experiments.lowprec_accuracy/1"))
      .add("identity", Json::text(identity(c)))
      .add("case", Json::text(case_name(c)))
      .add("spec_sha256", Json::text(kSpecSha256))
      .add("device", Json::text(props.name))
      .add("weight_conversion_ms_median_of_5", Json::real(weight_ms))
      .add("datasets", std::move(datasets))
      .add("status", Json::text("accuracy"));
  const std::string line = result.dump();
  if (record) *record = line;
  if (print) std::printf("RESULT %s\n", line.c_str());
  if (!json_out.empty()) {
    FILE *file = std::fopen(json_out.c_str(), "w");
    const bool written = file && std::fprintf(file, "%s\n", line.c_str()) >= 0;
    if (!(file && std::fclose(file) == 0 && written))
      appproto::abort_run(appproto::kUsage, "cannot write %s", json_out.c_str());
  }
  return appproto::kPass;
}

const appproto::Provenance kBuild{"gfx950", kSpecSha256, "v1", "4a75f8d743ef7fe755822bab0ea0fb78009c145b"};

// --accuracy and --selftest anywhere on the command line select those modes;
// anything else is the loom_private protocol.
int dispatch(int c, int argc, const char *const *argv, std::string *record, bool print) {
  if (c < kFp32 || c > kNvfp4) {
    std::fprintf(stderr, "lowprec: case must be 0 (fp32), 1 (bf16), 2 (mxfp6) or 3 (nvfp4) (got %d)\n", c);
    return appproto::kUsage;
  }
  appproto::set_program(kProgram);
  g_case = c;
  const auto has = [&](const char *flag) {
    return std::any_of(argv + 1, argv + argc, [&](const char *a) { return std::strcmp(a, flag) == 0; });
  };
  try {
    if (has("--accuracy")) return run_accuracy(c, argc, argv, record, print);
    if (has("--selftest")) return run_selftest(c);
  } catch (const appproto::Abort &a) {
    std::fprintf(stderr, "%s: %s\n", appproto::program(), a.what());
    return a.code();
  }
  return appproto::run_protocol(kProgram, argc, argv, protocol_factory, kBuild, record, print);
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
