// The loom_private application protocol, as this build's applications (the
// llama2c decoder and the lowprec classifier cases) present it: one command
// line, three actions (check, bench, profile), two launch forms (direct
// enqueue or one captured hipGraph), and one JSON result record.
//
// What callers and scripts rely on is the observable surface of
// applications/loom_private/common/lp_harness.cuh: option names and defaults
// (:1-40), exit codes (:17-18, 92-96), the stderr lines the decoder's
// tests/run_tests.sh greps, and the record schema. The structure below is
// this build's own.
//
//   --preset large                 the only preset outside tests (default)
//   --launch direct|graph|both     both (the default) is valid for check only
//   --action check|bench|profile   check is the default
//   --iterations N --warmup W      bench and profile (defaults 20 and 3)
//   --set key=value                dimension override, check only
//   --asset name=path              application asset path override
//   --json-out PATH                also write the record to PATH
//
// Errors never end the process: they throw Abort, and run_protocol turns it
// into the exit code after printing "<program>: <message>" to stderr, so the
// protocol also runs in-process from a library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace appproto {

// Process exit codes of the protocol.
enum Exit : int { kPass = 0, kMismatch = 1, kUsage = 2, kAsset = 3, kHipError = 70 };

// A run that cannot continue: its exit code and the one-line reason.
class Abort : public std::runtime_error {
 public:
  Abort(int code, const std::string &reason) : std::runtime_error(reason), code_(code) {}
  int code() const { return code_; }

 private:
  int code_;
};

// printf-style Abort.
[[noreturn]] void abort_run(int code, const char *format, ...) __attribute__((format(printf, 2, 3)));

// Name that prefixes every diagnostic line of the running program.
void set_program(const std::string &name);
const char *program();

// HIP / l2c calls inside applications: any failure aborts with kHipError.
void hip_check(hipError_t error, const char *what, const char *file, int line);
#define APP_HIP(call) ::appproto::hip_check((call), #call, __FILE__, __LINE__)
#define APP_L2C(call) ::appproto::hip_check(static_cast<hipError_t>(call), #call, __FILE__, __LINE__)

// 64-bit FNV-1a over byte ranges: compares invocations and launch forms
// (not a cryptographic hash).
class Digest {
 public:
  Digest &add(const void *data, size_t bytes);
  uint64_t value() const { return state_; }
  static std::string hex(uint64_t value);

 private:
  uint64_t state_ = 0xcbf29ce484222325ull;
};

// A small JSON value with objects that keep insertion order.
class Json {
 public:
  Json() = default;  // null
  static Json text(const std::string &s);
  static Json real(double v);  // non-finite values become null
  static Json whole(long long v);
  static Json flag(bool v);
  static Json object();
  static Json list();
  Json &add(const std::string &key, Json value);  // objects
  Json &push(Json value);                         // lists
  std::string dump() const;

 private:
  enum class Kind { kNull, kText, kNumber, kFlag, kObject, kList };
  Kind kind_ = Kind::kNull;
  std::string scalar_;  // text, or the number's / flag's literal
  std::vector<std::pair<std::string, Json>> members_;
  std::vector<Json> items_;
  void write(std::string *out) const;
};

// The --set values an application may read. Each read consumes its key;
// whatever is left unread afterwards is an unsupported key.
class Settings {
 public:
  void put(const std::string &key, const std::string &value) { pending_[key] = value; }
  bool empty() const { return pending_.empty(); }
  long long integer(const std::string &key, long long fallback);
  // First key nobody read, or "".
  std::string unread() const { return pending_.empty() ? std::string() : pending_.begin()->first; }
  // The keys read, with their values, in reading order.
  Json applied() const;

 private:
  std::map<std::string, std::string> pending_;
  std::vector<std::pair<std::string, long long>> used_;
};

// The --asset paths. Applications ask by name; a name given on the command
// line that no application asked for is an error.
class Assets {
 public:
  void put(const std::string &name, const std::string &path) { given_[name] = path; }
  std::string path(const std::string &name, const std::string &fallback);
  std::string unclaimed() const;

 private:
  std::map<std::string, std::string> given_;
  std::vector<std::string> claimed_;
};

// Which work one enqueue covers: the whole application (uploads and
// downloads included) or only the device compute.
enum class Scope { kApplication, kCompute };

// What an application says about itself in the record.
struct AppInfo {
  std::string identity;
  Json dimensions = Json::object();
  Json asset_sha256 = Json::object();
  std::string application_scope, compute_scope;
};

// One application under the protocol. enqueue() must be capture-safe: no
// synchronization, no allocation and no host logic that depends on device
// results, and host buffers that cross PCIe are pinned (hipHostMalloc).
class Application {
 public:
  virtual ~Application() = default;
  virtual AppInfo info() const = 0;
  // Allocations, uploads and weight preparation (untimed).
  virtual void prepare(hipStream_t stream) = 0;
  virtual void enqueue(Scope scope, hipStream_t stream) = 0;
  // Fills every output (device and host copies) with 0xFF bytes.
  virtual void scramble_outputs(hipStream_t stream) = 0;
  // The CPU expectation of the check action.
  virtual void derive_expected() = 0;
  // Downloads the diagnostics and compares them with the expectation,
  // printing the first mismatches.
  virtual bool outputs_match() = 0;
  virtual uint64_t outputs_digest() const = 0;
};

// Builds the application for a preset, reading its --set and --asset values;
// null for an unknown preset. Invalid dimensions abort with kUsage.
using AppFactory = std::function<std::unique_ptr<Application>(const std::string &preset, Settings &settings,
                                                             Assets &assets)>;

// Fixed record fields of a build.
struct Provenance {
  std::string variant;          // e.g. "gfx950"
  std::string contract_sha256;  // of the contract the application implements
  std::string suite_version;
  std::string loom_commit;
};

// The whole program: reads argv, runs the action, prints "RESULT <json>" on
// stdout when `print` is set, writes --json-out, and returns the exit code.
// *record receives the record ("" when the run ended before it was built).
int run_protocol(const std::string &program_name, int argc, const char *const *argv, const AppFactory &factory,
                 const Provenance &provenance, std::string *record, bool print);

}  // namespace appproto
