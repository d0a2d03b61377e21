// The loom_private application protocol (app_protocol.h).
//
// Layout: diagnostics and small value types first (Abort, Digest, Json,
// Settings, Assets), then the command line (a table of options read in two
// passes: shape, then meaning), the launch forms (Replay), the timing of a
// scope, and finally the three actions and the record.
#include "app_protocol.h"

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#if __has_include(<rocprofiler-sdk-roctx/roctx.h>)
#include <rocprofiler-sdk-roctx/roctx.h>
#define APP_HAVE_ROCTX 1
#else
#define APP_HAVE_ROCTX 0
#endif

namespace appproto {

// ---------------------------------------------------------------------------
// Diagnostics.

namespace {
std::string &program_storage() {
  static std::string name = "app";
  return name;
}

std::string vformat(const char *format, va_list args) {
  va_list copy;
  va_copy(copy, args);
  const int n = std::vsnprintf(nullptr, 0, format, copy);
  va_end(copy);
  std::string out(n > 0 ? static_cast<size_t>(n) : 0, '\0');
  if (n > 0) std::vsnprintf(&out[0], out.size() + 1, format, args);
  return out;
}

double seconds_between(std::chrono::steady_clock::time_point a) {
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - a).count();
}
}  // namespace

void set_program(const std::string &name) { program_storage() = name; }
const char *program() { return program_storage().c_str(); }

void abort_run(int code, const char *format, ...) {
  va_list args;
  va_start(args, format);
  std::string reason = vformat(format, args);
  va_end(args);
  throw Abort(code, reason);
}

void hip_check(hipError_t error, const char *what, const char *file, int line) {
  if (error != hipSuccess)
    abort_run(kHipError, "%s:%d: %s failed: %s", file, line, what, hipGetErrorString(error));
}

// ---------------------------------------------------------------------------
// Digest and JSON.

Digest &Digest::add(const void *data, size_t bytes) {
  constexpr uint64_t kPrime = 0x100000001b3ull;
  const unsigned char *p = static_cast<const unsigned char *>(data);
  for (const unsigned char *end = p + bytes; p != end; ++p) state_ = (state_ ^ *p) * kPrime;
  return *this;
}

std::string Digest::hex(uint64_t value) {
  static const char kDigits[] = "0123456789abcdef";
  std::string s(16, '0');
  for (int i = 15; i >= 0; --i, value >>= 4) s[static_cast<size_t>(i)] = kDigits[value & 15u];
  return s;
}

Json Json::text(const std::string &s) {
  Json j;
  j.kind_ = Kind::kText;
  j.scalar_ = s;
  return j;
}

Json Json::real(double v) {
  if (!std::isfinite(v)) return Json();
  char buf[40];
  std::snprintf(buf, sizeof buf, "%.10g", v);
  Json j;
  j.kind_ = Kind::kNumber;
  j.scalar_ = buf;
  return j;
}

Json Json::whole(long long v) {
  Json j;
  j.kind_ = Kind::kNumber;
  j.scalar_ = std::to_string(v);
  return j;
}

Json Json::flag(bool v) {
  Json j;
  j.kind_ = Kind::kFlag;
  j.scalar_ = v ? "true" : "false";
  return j;
}

Json Json::object() {
  Json j;
  j.kind_ = Kind::kObject;
  return j;
}

Json Json::list() {
  Json j;
  j.kind_ = Kind::kList;
  return j;
}

Json &Json::add(const std::string &key, Json value) {
  members_.emplace_back(key, std::move(value));
  return *this;
}

Json &Json::push(Json value) {
  items_.push_back(std::move(value));
  return *this;
}

namespace {
void write_string(const std::string &s, std::string *out) {
  out->push_back('"');
  for (const char ch : s) {
    const unsigned char c = static_cast<unsigned char>(ch);
    if (c == '"' || c == '\\') {
      out->push_back('\\');
      out->push_back(ch);
    } else if (c >= 0x20) {
      out->push_back(ch);
    } else if (c == '\n') {
      *out += "\\n";
    } else if (c == '\t') {
      *out += "\\t";
    } else {
      char esc[8];
      std::snprintf(esc, sizeof esc, "\\u%04x", c);
      *out += esc;
    }
  }
  out->push_back('"');
}
}  // namespace

void Json::write(std::string *out) const {
  switch (kind_) {
    case Kind::kNull: *out += "null"; return;
    case Kind::kText: write_string(scalar_, out); return;
    case Kind::kNumber:
    case Kind::kFlag: *out += scalar_; return;
    case Kind::kObject: {
      out->push_back('{');
      const char *sep = "";
      for (const auto &m : members_) {
        *out += sep;
        write_string(m.first, out);
        *out += ": ";
        m.second.write(out);
        sep = ", ";
      }
      out->push_back('}');
      return;
    }
    case Kind::kList: {
      out->push_back('[');
      for (size_t i = 0; i < items_.size(); ++i) {
        if (i) *out += ", ";
        items_[i].write(out);
      }
      out->push_back(']');
      return;
    }
  }
}

std::string Json::dump() const {
  std::string out;
  write(&out);
  return out;
}

// ---------------------------------------------------------------------------
// --set and --asset values.

long long Settings::integer(const std::string &key, long long fallback) {
  const auto found = pending_.find(key);
  if (found == pending_.end()) return fallback;
  const std::string text = found->second;
  errno = 0;
  char *end = nullptr;
  const long long v = std::strtoll(text.c_str(), &end, 0);
  if (text.empty() || errno != 0 || *end != '\0')
    abort_run(kUsage, "--set %s=%s is not an integer", key.c_str(), text.c_str());
  pending_.erase(found);
  used_.emplace_back(key, v);
  return v;
}

Json Settings::applied() const {
  Json j = Json::object();
  for (const auto &kv : used_) j.add(kv.first, Json::whole(kv.second));
  return j;
}

std::string Assets::path(const std::string &name, const std::string &fallback) {
  claimed_.push_back(name);
  const auto found = given_.find(name);
  return found == given_.end() ? fallback : found->second;
}

std::string Assets::unclaimed() const {
  for (const auto &kv : given_)
    if (std::find(claimed_.begin(), claimed_.end(), kv.first) == claimed_.end()) return kv.first;
  return std::string();
}

// ---------------------------------------------------------------------------
// Command line.

namespace {

enum class Action { kCheck, kBench, kProfile };
constexpr unsigned kDirectForm = 1u, kGraphForm = 2u;

const char *action_name(Action a) {
  return a == Action::kCheck ? "check" : a == Action::kBench ? "bench" : "profile";
}
const char *forms_name(unsigned forms) {
  return forms == kDirectForm ? "direct" : forms == kGraphForm ? "graph" : "both";
}

struct Request {
  std::string preset = "large";
  unsigned forms = kDirectForm | kGraphForm;
  bool forms_given = false;
  Action action = Action::kCheck;
  int iterations = 20;
  int warmup = 3;
  Settings settings;
  Assets assets;
  std::string record_path;
};

enum class Opt { kPreset, kLaunch, kAction, kIterations, kWarmup, kSet, kAsset, kJsonOut };
struct OptionName {
  const char *flag;
  Opt opt;
};
constexpr OptionName kOptions[] = {
    {"--preset", Opt::kPreset}, {"--launch", Opt::kLaunch},   {"--action", Opt::kAction},
    {"--iterations", Opt::kIterations}, {"--warmup", Opt::kWarmup}, {"--set", Opt::kSet},
    {"--asset", Opt::kAsset},   {"--json-out", Opt::kJsonOut},
};

void print_usage() {
  std::printf(
      "usage: %s [--preset large] [--launch direct|graph|both]\n"
      "          [--action check|bench|profile] [--iterations N] [--warmup W]\n"
      "          [--set key=value]... [--asset name=path]... [--json-out PATH]\n"
      "Defaults: --preset large --action check --launch both.\n"
      "bench and profile need an explicit --launch direct or --launch graph.\n",
      program());
}

int count_value(const char *flag, const std::string &text, int lowest) {
  char *end = nullptr;
  errno = 0;
  const long v = std::strtol(text.c_str(), &end, 10);
  if (text.empty() || errno != 0 || *end != '\0' || v < lowest || v > 1000000)
    abort_run(kUsage, "%s expects an integer >= %d, got '%s'", flag, lowest, text.c_str());
  return static_cast<int>(v);
}

std::pair<std::string, std::string> key_value(const char *flag, const std::string &text) {
  const size_t eq = text.find('=');
  if (eq == std::string::npos || eq == 0) abort_run(kUsage, "%s expects key=value, got '%s'", flag, text.c_str());
  return {text.substr(0, eq), text.substr(eq + 1)};
}

// Pass 1 checks the shape (known flags, each with a value); pass 2 gives
// the values their meaning. Returns false for --help (already printed).
bool read_command_line(int argc, const char *const *argv, Request *rq) {
  std::vector<std::pair<Opt, std::string>> given;
  for (int i = 1; i < argc; ++i) {
    const std::string flag = argv[i];
    if (flag == "--help" || flag == "-h") {
      print_usage();
      return false;
    }
    const OptionName *match = nullptr;
    for (const OptionName &o : kOptions)
      if (flag == o.flag) match = &o;
    if (!match) abort_run(kUsage, "unknown option %s (see --help)", flag.c_str());
    if (i + 1 >= argc) abort_run(kUsage, "%s needs a value", flag.c_str());
    given.emplace_back(match->opt, argv[++i]);
  }
  for (const auto &entry : given) {
    const std::string &v = entry.second;
    switch (entry.first) {
      case Opt::kPreset: rq->preset = v; break;
      case Opt::kLaunch:
        if (v == "direct") rq->forms = kDirectForm;
        else if (v == "graph") rq->forms = kGraphForm;
        else if (v == "both") rq->forms = kDirectForm | kGraphForm;
        else abort_run(kUsage, "--launch must be direct, graph or both");
        rq->forms_given = true;
        break;
      case Opt::kAction:
        if (v == "check") rq->action = Action::kCheck;
        else if (v == "bench") rq->action = Action::kBench;
        else if (v == "profile") rq->action = Action::kProfile;
        else abort_run(kUsage, "--action must be check, bench or profile");
        break;
      case Opt::kIterations: rq->iterations = count_value("--iterations", v, 1); break;
      case Opt::kWarmup: rq->warmup = count_value("--warmup", v, 0); break;
      case Opt::kSet: {
        const auto kv = key_value("--set", v);
        rq->settings.put(kv.first, kv.second);
        break;
      }
      case Opt::kAsset: {
        const auto kv = key_value("--asset", v);
        rq->assets.put(kv.first, kv.second);
        break;
      }
      case Opt::kJsonOut: rq->record_path = v; break;
    }
  }
  if (rq->action != Action::kCheck) {
    if (!rq->forms_given || rq->forms == (kDirectForm | kGraphForm))
      abort_run(kUsage, "%s needs --launch direct or --launch graph", action_name(rq->action));
    if (!rq->settings.empty()) abort_run(kUsage, "--set is only valid with --action check");
  }
  return true;
}

// ---------------------------------------------------------------------------
// Launch forms: the body enqueued directly, or captured once into a graph and
// replayed.

class Replay {
 public:
  Replay(bool as_graph, hipStream_t stream, std::function<void()> body)
      : stream_(stream), body_(std::move(body)) {
    if (!as_graph) return;
    hipGraph_t graph = nullptr;
    APP_HIP(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
    body_();
    APP_HIP(hipStreamEndCapture(stream_, &graph));
    const hipError_t made = hipGraphInstantiate(&exec_, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    APP_HIP(made);
    APP_HIP(hipGraphUpload(exec_, stream_));
    APP_HIP(hipStreamSynchronize(stream_));
  }
  ~Replay() {
    if (exec_) (void)hipGraphExecDestroy(exec_);
  }
  Replay(const Replay &) = delete;
  Replay &operator=(const Replay &) = delete;

  void operator()() {
    if (exec_) APP_HIP(hipGraphLaunch(exec_, stream_));
    else body_();
  }

 private:
  hipStream_t stream_;
  std::function<void()> body_;
  hipGraphExec_t exec_ = nullptr;
};

// ---------------------------------------------------------------------------
// Timing of one scope: warm-up launches, one back-to-back batch between two
// events, then as many single launches from an idle device.

class EventPair {
 public:
  EventPair() {
    APP_HIP(hipEventCreate(&start_));
    APP_HIP(hipEventCreate(&stop_));
  }
  ~EventPair() {
    (void)hipEventDestroy(start_);
    (void)hipEventDestroy(stop_);
  }
  EventPair(const EventPair &) = delete;
  EventPair &operator=(const EventPair &) = delete;
  void start(hipStream_t s) { APP_HIP(hipEventRecord(start_, s)); }
  double stop_ms(hipStream_t s) {
    APP_HIP(hipEventRecord(stop_, s));
    APP_HIP(hipEventSynchronize(stop_));
    float ms = 0.0f;
    APP_HIP(hipEventElapsedTime(&ms, start_, stop_));
    return ms;
  }

 private:
  hipEvent_t start_ = nullptr, stop_ = nullptr;
};

struct ScopeTiming {
  double batch_ms = 0.0;
  int iterations = 0;
  std::vector<double> singles_us;
};

ScopeTiming time_scope(Replay &replay, hipStream_t stream, int warmup, int iterations) {
  ScopeTiming t;
  t.iterations = iterations;
  for (int i = 0; i < warmup; ++i) replay();
  APP_HIP(hipStreamSynchronize(stream));
  EventPair events;
  events.start(stream);
  for (int i = 0; i < iterations; ++i) replay();
  t.batch_ms = events.stop_ms(stream);
  for (int i = 0; i < iterations; ++i) {
    APP_HIP(hipDeviceSynchronize());
    events.start(stream);
    replay();
    t.singles_us.push_back(1000.0 * events.stop_ms(stream));
  }
  return t;
}

double middle_value(std::vector<double> v) {
  if (v.empty()) return 0.0;
  const size_t half = v.size() / 2;
  std::nth_element(v.begin(), v.begin() + static_cast<long>(half), v.end());
  const double upper = v[half];
  if (v.size() % 2) return upper;
  return 0.5 * (upper + *std::max_element(v.begin(), v.begin() + static_cast<long>(half)));
}

Json timing_json(const ScopeTiming &t, const std::string &scope) {
  Json singles = Json::list();
  for (double us : t.singles_us) singles.push(Json::real(us));
  Json j = Json::object();
  j.add("scope", Json::text(scope));
  j.add("batch_total_ms", Json::real(t.batch_ms));
  j.add("batch_per_iteration_us", Json::real(1000.0 * t.batch_ms / t.iterations));
  j.add("single_median_us", Json::real(middle_value(t.singles_us)));
  j.add("single_us", std::move(singles));
  return j;
}

struct OwnedStream {
  hipStream_t s = nullptr;
  OwnedStream() { APP_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking)); }
  ~OwnedStream() {
    if (s) (void)hipStreamDestroy(s);
  }
};

// ---------------------------------------------------------------------------
// Actions.

// check: the expectation, then two invocations per launch form, each from
// scrambled outputs; every invocation must match and all digests agree.
bool check_action(Application &app, hipStream_t stream, unsigned forms, Json *record) {
  auto clock = std::chrono::steady_clock::now();
  app.derive_expected();
  std::fprintf(stderr, "%s: CPU oracle %.2f s\n", program(), seconds_between(clock));
  Json checks = Json::list();
  std::vector<uint64_t> digests;
  bool every_pass = true;
  for (const unsigned form : {kDirectForm, kGraphForm}) {
    if (!(forms & form)) continue;
    Replay replay(form == kGraphForm, stream, [&] { app.enqueue(Scope::kApplication, stream); });
    for (int invocation = 1; invocation <= 2; ++invocation) {
      app.scramble_outputs(stream);
      APP_HIP(hipStreamSynchronize(stream));
      clock = std::chrono::steady_clock::now();
      replay();
      APP_HIP(hipStreamSynchronize(stream));
      APP_HIP(hipGetLastError());
      const double secs = seconds_between(clock);
      const bool pass = app.outputs_match();
      const uint64_t digest = app.outputs_digest();
      digests.push_back(digest);
      every_pass = every_pass && pass;
      std::fprintf(stderr, "%s: %s invocation %d: %s, digest %s (%.2f s, untimed)\n", program(), forms_name(form),
                   invocation, pass ? "PASS" : "FAIL", Digest::hex(digest).c_str(), secs);
      Json c = Json::object();
      c.add("launch", Json::text(forms_name(form)));
      c.add("invocation", Json::whole(invocation));
      c.add("pass", Json::flag(pass));
      c.add("digest", Json::text(Digest::hex(digest)));
      checks.push(std::move(c));
    }
  }
  const bool agree = std::all_of(digests.begin(), digests.end(), [&](uint64_t d) { return d == digests.front(); });
  if (!agree) std::fprintf(stderr, "%s: FAIL: invocations or launch modes disagree\n", program());
  const bool pass = every_pass && agree;
  record->add("checks", std::move(checks));
  record->add("outputs_agree", Json::flag(agree));
  record->add("timing", Json());
  record->add("status", Json::text(pass ? "pass" : "fail"));
  return pass;
}

// profile: one warm-up invocation, then one inside the profiler's selected
// region (rocprofv3 --selected-regions follows the roctx resume/pause pair).
void profile_action(Application &app, hipStream_t stream, unsigned forms, Json *record) {
  Replay replay(forms == kGraphForm, stream, [&] { app.enqueue(Scope::kApplication, stream); });
  replay();
  APP_HIP(hipStreamSynchronize(stream));
#if APP_HAVE_ROCTX
  roctx_thread_id_t tid = 0;
  roctxGetThreadId(&tid);
  roctxProfilerResume(tid);
  roctxRangePushA("lp.profile");
#endif
  replay();
  APP_HIP(hipStreamSynchronize(stream));
#if APP_HAVE_ROCTX
  roctxRangePop();
  roctxProfilerPause(tid);
#endif
  record->add("profiled", Json::text("one application-scope invocation after one warmup invocation"));
  record->add("timing", Json());
  record->add("output_digest", Json::text(Digest::hex(app.outputs_digest())));
  record->add("status", Json::text("profile"));
}

// bench: the application scope, then the compute scope, each timed alone.
void bench_action(Application &app, const AppInfo &info, hipStream_t stream, const Request &rq, Json *record) {
  const bool graph = rq.forms == kGraphForm;
  Json timing = Json::object();
  {
    Replay replay(graph, stream, [&] { app.enqueue(Scope::kApplication, stream); });
    timing.add("application", timing_json(time_scope(replay, stream, rq.warmup, rq.iterations),
                                          info.application_scope));
  }
  {
    Replay replay(graph, stream, [&] { app.enqueue(Scope::kCompute, stream); });
    timing.add("compute", timing_json(time_scope(replay, stream, rq.warmup, rq.iterations), info.compute_scope));
  }
  APP_HIP(hipStreamSynchronize(stream));
  record->add("iterations", Json::whole(rq.iterations));
  record->add("warmup", Json::whole(rq.warmup));
  record->add("timing", std::move(timing));
  record->add("output_digest", Json::text(Digest::hex(app.outputs_digest())));
  record->add("status", Json::text("unvalidated_bench"));
}

void write_record_file(const std::string &path, const std::string &line) {
  FILE *f = std::fopen(path.c_str(), "w");
  bool ok = f != nullptr && std::fputs(line.c_str(), f) >= 0 && std::fputc('\n', f) != EOF;
  if (f != nullptr && std::fclose(f) != 0) ok = false;
  if (!ok) abort_run(kUsage, "cannot write %s", path.c_str());
}

int run_once(int argc, const char *const *argv, const AppFactory &factory, const Provenance &provenance,
             std::string *record_out, bool print) {
  Request rq;
  if (!read_command_line(argc, argv, &rq)) return kPass;
  std::unique_ptr<Application> app = factory(rq.preset, rq.settings, rq.assets);
  if (!app) abort_run(kUsage, "unknown preset '%s' (available: large)", rq.preset.c_str());
  if (!rq.settings.empty()) abort_run(kUsage, "unsupported --set key '%s'", rq.settings.unread().c_str());
  const std::string stray = rq.assets.unclaimed();
  if (!stray.empty()) abort_run(kUsage, "unsupported --asset name '%s'", stray.c_str());

  int device = 0, runtime = 0, driver = 0;
  hipDeviceProp_t props{};
  APP_HIP(hipGetDevice(&device));
  APP_HIP(hipGetDeviceProperties(&props, device));
  APP_HIP(hipRuntimeGetVersion(&runtime));
  APP_HIP(hipDriverGetVersion(&driver));

  OwnedStream owned;
  const auto clock = std::chrono::steady_clock::now();
  app->prepare(owned.s);
  APP_HIP(hipStreamSynchronize(owned.s));
  std::fprintf(stderr, "%s: setup %.2f s\n", program(), seconds_between(clock));

  const AppInfo info = app->info();
  Json device_json = Json::object();
  device_json.add("name", Json::text(props.name))
      .add("arch", Json::text(props.gcnArchName))
      .add("hip_runtime", Json::whole(runtime))
      .add("hip_driver", Json::whole(driver));
  Json scopes = Json::object();
  scopes.add("application", Json::text(info.application_scope)).add("compute", Json::text(info.compute_scope));
  Json record = Json::object();
  record.add("schema", Json::text("loom_private.result/1"))
      .add("suite_version", Json::text(provenance.suite_version))
      .add("identity", Json::text(info.identity))
      .add("variant", Json::text(provenance.variant))
      .add("loom_commit", Json::text(provenance.loom_commit))
      .add("contract_sha256", Json::text(provenance.contract_sha256))
      .add("preset", Json::text(rq.preset))
      .add("overrides", rq.settings.applied())
      .add("dimensions", info.dimensions)
      .add("asset_sha256", info.asset_sha256)
      .add("action", Json::text(action_name(rq.action)))
      .add("launch", Json::text(forms_name(rq.forms)))
      .add("device", std::move(device_json))
      .add("timing_scope", std::move(scopes));

  int code = kPass;
  switch (rq.action) {
    case Action::kCheck: code = check_action(*app, owned.s, rq.forms, &record) ? kPass : kMismatch; break;
    case Action::kProfile: profile_action(*app, owned.s, rq.forms, &record); break;
    case Action::kBench: bench_action(*app, info, owned.s, rq, &record); break;
  }

  const std::string line = record.dump();
  if (record_out) *record_out = line;
  if (print) {
    std::printf("RESULT %s\n", line.c_str());
    std::fflush(stdout);
  }
  if (!rq.record_path.empty()) write_record_file(rq.record_path, line);
  return code;
}

}  // namespace

int run_protocol(const std::string &program_name, int argc, const char *const *argv, const AppFactory &factory,
                 const Provenance &provenance, std::string *record, bool print) {
  set_program(program_name);
  if (record) record->clear();
  try {
    return run_once(argc, argv, factory, provenance, record, print);
  } catch (const Abort &a) {
    std::fprintf(stderr, "%s: %s\n", program(), a.what());
    std::fflush(stderr);
    return a.code();
  }
}

}  // namespace appproto
