// The loom_private application protocol on HIP: command line, direct and
// hipGraph executors, the poison / two-invocation / digest check, timing and
// the one-line JSON result record. Restates the behaviour of
// applications/loom_private/common/lp_harness.cuh:1-596 for this build's
// applications (the llama2c decoder).
//
//   --preset large            the only preset outside tests (default)
//   --launch direct|graph|both  both is the default and only valid for check
//   --action check|bench|profile  check is the default
//   --iterations N --warmup W bench only (defaults 20 and 3)
//   --set key=value           dimension override, check only
//   --asset name=path         application asset path override
//   --json-out PATH           also write the result record to PATH
//
// Exit codes: 0 pass, 1 output mismatch, 2 usage or invalid dimensions,
// 3 missing or corrupt asset, 70 HIP error (lp_harness.cuh:17-18,92-96).
//
// Errors do not end the process: fail() throws lp::Exit, which run_main turns
// into its return value, so the protocol also runs in-process from a library
// (l2c_decoder_main).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace lp {

constexpr int kExitPass = 0;
constexpr int kExitMismatch = 1;
constexpr int kExitUsage = 2;
constexpr int kExitAsset = 3;
constexpr int kExitHip = 70;

// Thrown by fail(); carries the exit code. The message is already printed.
struct Exit {
  int code;
};

// Prints "<app>: <message>" to stderr and throws Exit{code}.
[[noreturn]] void fail(int code, const char *format, ...) __attribute__((format(printf, 2, 3)));

// Name used as the prefix of every diagnostic line.
void set_app_name(const std::string &name);
const std::string &app_name();

#define LP_HIP(call)                                                                          \
  do {                                                                                        \
    const hipError_t lp_error_ = (call);                                                      \
    if (lp_error_ != hipSuccess)                                                              \
      ::lp::fail(::lp::kExitHip, "%s:%d: %s failed: %s", __FILE__, __LINE__, #call,           \
                 hipGetErrorString(lp_error_));                                               \
  } while (0)

// Return code of an l2c_* C-ABI call (a hipError_t value).
#define LP_L2C(call)                                                                          \
  do {                                                                                        \
    const int lp_code_ = (call);                                                              \
    if (lp_code_ != 0)                                                                        \
      ::lp::fail(::lp::kExitHip, "%s:%d: %s failed: %s", __FILE__, __LINE__, #call,           \
                 hipGetErrorString(static_cast<hipError_t>(lp_code_)));                       \
  } while (0)

// FNV-1a 64 over bytes (compares invocations and launch modes; not a
// cryptographic hash).
uint64_t fnv1a64(const void *data, size_t bytes, uint64_t state = 1469598103934665603ull);
std::string hex64(uint64_t value);

// Ordered key -> raw JSON text.
using JsonObject = std::vector<std::pair<std::string, std::string>>;
namespace json {
std::string quote(const std::string &text);
std::string number(double value);
std::string integer(long long value);
std::string boolean(bool value);
std::string render(const JsonObject &object);
}  // namespace json

enum class Launch { Direct, Graph, Both };
enum class Action { Check, Bench, Profile };
const char *name(Launch launch);

struct Options {
  std::string preset = "large";
  Launch launch = Launch::Both;
  bool launch_given = false;
  Action action = Action::Check;
  int iterations = 20;
  int warmup = 3;
  std::map<std::string, std::string> overrides;  // --set
  std::map<std::string, std::string> assets;     // --asset
  std::string json_out;

  // Integer dimension from --set (removed from the unconsumed set), else the
  // fallback.
  long long take_int(const std::string &key, long long fallback);
  // Asset path from --asset, else the fallback; marks the name as known.
  std::string asset(const std::string &key, const std::string &fallback);
  const std::vector<std::pair<std::string, std::string>> &consumed() const { return consumed_; }
  // First --asset name that no asset() call asked for, or "".
  std::string unknown_asset() const;

 private:
  std::vector<std::pair<std::string, std::string>> consumed_;
  std::vector<std::string> assets_known_;
};

// One application. Host buffers that cross PCIe in enqueue_application are
// pinned (hipHostMalloc) so the work can be captured into a hipGraph;
// enqueue_* is capture-safe (no synchronization, allocation or host logic
// that depends on device results).
class Workload {
 public:
  virtual ~Workload() = default;
  virtual std::string identity() const = 0;
  virtual JsonObject dimensions() const = 0;
  virtual JsonObject asset_hashes() const { return {}; }
  virtual std::string application_scope() const = 0;
  virtual std::string compute_scope() const = 0;
  virtual void setup(hipStream_t stream) = 0;
  virtual void enqueue_application(hipStream_t stream) = 0;
  virtual void enqueue_compute(hipStream_t stream) = 0;
  virtual void poison_outputs(hipStream_t stream) = 0;
  virtual void compute_reference() = 0;
  virtual bool check_outputs() = 0;
  virtual uint64_t output_digest() const = 0;
};

// Builds the workload for the parsed options, or returns null for an unknown
// preset. Invalid dimensions call fail(kExitUsage, ...).
using Factory = std::unique_ptr<Workload> (*)(Options &options);

struct Build {
  std::string variant;          // e.g. "gfx950"
  std::string contract_sha256;  // sha256 of the application's contract
  std::string suite_version;
  std::string loom_commit;
};

// The whole program: parses argv, runs the action, prints "RESULT <json>" to
// stdout (when print is set) and returns the exit code. *record receives the
// JSON record (empty when the run ended before it was built).
int run_main(int argc, const char *const *argv, Factory factory, const Build &build,
             std::string *record, bool print);

}  // namespace lp
