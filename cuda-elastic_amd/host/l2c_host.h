// Host side of the llama2c harness: options, input generation, the CPU
// validation rules, the dump format and the iteration runner.
//
// This is the drop-in process surface of the reference binaries
// llama2c/llama2c_cuda_graph.cu and llama2c/llama2c_sota.cu (one command line,
// one key=value output line, exit code 0/1) re-designed for HIP on MI355X.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace l2c_host {

constexpr float kRmsEpsilon = 1.0e-5f;  // llama2c/llama2c_common.h:44

// Input modes. deterministic and random follow llama2c/llama2c_common.h:105-132;
// scaled and normal carry the benchmark-configuration distributions.
enum class InputMode : int32_t {
  kDeterministic = 0,  // 1,2,3,4 repeating; weight 1; shifted identity matrix
  kRandom = 1,         // every stream U[-1,1) on a 2^-23 grid
  kScaled = 2,         // x, logits U[-1,1); weight 1 + u/2 in [0.5,1.5); W = u / sqrt(size)
  kNormal = 3,         // as scaled, but W = N(0,1) / sqrt(size) (Box-Muller)
};

// Matrix product variants (the reference's `naive|coalesced` token plus the
// variants this build adds).
enum class Matmul : int32_t {
  kNaive = 0,      // matvec on input[0], one lane per row
  kCoalesced = 1,  // matvec on input[0], one wavefront per row
  kFused = 2,      // one launch for the whole iteration (llama2c_sota.cu design)
  kBatched = 3,    // out[b][r] = sum_k W[r][k] x[b][k] on fp32 MFMA
  kMxfp4 = 4,      // batched, bf16 activations x MXFP4 weights
  kFp8 = 5,        // batched, bf16 activations x per-row-scaled fp8 e4m3 weights
  kMxfp4s = 6,     // mxfp4 weights on the block-scaled matrix cores, MXFP8 activations
  kFp8s = 7,       // fp8 weights on the block-scaled matrix cores, MXFP8 activations
};

const char *matmul_name(Matmul m);
const char *input_name(InputMode m);
inline bool matmul_is_scaled(Matmul m) { return m == Matmul::kMxfp4s || m == Matmul::kFp8s; }
inline bool matmul_is_quantized(Matmul m) {
  return m == Matmul::kMxfp4 || m == Matmul::kFp8 || matmul_is_scaled(m);
}
inline bool matmul_is_batched(Matmul m) { return m == Matmul::kBatched || matmul_is_quantized(m); }
// MXFP4 weights (else per-row fp8) for a quantized variant.
inline bool matmul_is_mxfp4(Matmul m) { return m == Matmul::kMxfp4 || m == Matmul::kMxfp4s; }

struct InputOptions {
  InputMode mode = InputMode::kDeterministic;
  uint64_t seed = 0;
  std::string dump_path;
};

// Defaults: llama2c/llama2c_cuda_graph.cu:43-53,178-193.
struct Options {
  bool graph = true;
  int launches = 180;
  int batch = 512;
  int size = 16384;
  int rows = 8192;
  int repeats = 1;
  int warmup_ms = 100;
  bool copy_outputs = true;
  Matmul matmul = Matmul::kNaive;
  bool auto_launches = false;
  bool full_check = false;  // validate every (b, r) of a batched product
  int warmup_iters = 0;     // > 0: at least this many warm-up iterations, and at least warmup_ms
  // Iteration forms beyond the reference protocol (llama2c_cuda_graph.cu:347-381):
  bool one_stream = false;  // every launch and copy on one stream, no fork/join events
  bool host_write = false;  // copy mode: a device kernel stores the outputs into the
                            // pinned host buffers in place of hipMemcpyAsync
  int device = 0;
  InputOptions inputs;
};

// Parses argv like llama2c/llama2c_cuda_graph.cu:211-258 (keyword tokens
// anywhere, positionals in order, `auto` only as the first positional) plus
// LLAMA2C_DUMP (llama2c/llama2c_common.h:84-88). Returns false on a usage
// error; writes a message to *error for a malformed seed.
bool parse_options(int argc, const char *const *argv, Options *options, std::string *error);
std::string usage_text(const char *program);

// ---------------------------------------------------------------------------
// Inputs

uint64_t splitmix64(uint64_t x);
// Counter-based uniform on [-1, 1), 2^-23 grid (llama2c/llama2c_common.h:92-103).
float uniform(uint64_t seed, uint64_t stream, uint64_t index);
// Standard normal number i of the stream (seed * 0x100000001b3 + stream) in the
// sequential splitmix64 + Box-Muller recipe of
// experiments/blackwell/lowprec/spec.json:49, rounded to float.
float normal(uint64_t seed, uint64_t stream, uint64_t index);

struct Inputs {
  std::vector<float> input;          // batch x size
  std::vector<float> probabilities;  // batch x size (the softmax logits)
  std::vector<float> weight;         // size
  std::vector<float> matrix;         // rows x size
};

// Fills with `threads` host threads (0 = all usable cores).
void fill_inputs(const InputOptions &options, int batch, int size, int rows, Inputs *inputs,
                 int threads = 0);

// ---------------------------------------------------------------------------
// Quantized weight formats (host encoders; the device quantizers must match
// them bit for bit).

uint16_t bf16_bits(float v);             // round to nearest even
float bf16_value(uint16_t bits);
float e2m1_value(unsigned code);         // code 0..15, bit 3 = sign
unsigned e2m1_encode(double v);          // nearest, ties to even code, saturating, -0 -> 0
float e4m3_value(unsigned code);         // OCP e4m3fn, bias 7
unsigned e4m3_encode(float v);           // nearest even, saturating at 448
int mxfp4_block_exponent(float amax);    // floor(log2(amax / 6)) clamped to [-127, 127]
int mxfp8_block_exponent(float amax);    // ceil(log2(amax / 448)) clamped to [-127, 127]

// ---------------------------------------------------------------------------
// Validation (restates llama2c/llama2c_common.h:139-319 and extends it to
// batched and quantized products).

double gamma_probabilistic(int n);  // llama2c/llama2c_common.h:231-235

struct ProductCheck {
  // One entry per checked product element (rows for a matvec; batch x rows
  // for a batched product, NaN where a row of the batch was not sampled).
  std::vector<float> tolerance;
  std::vector<double> reference;
  std::vector<int> sampled_batch_rows;  // batched products only
};

struct Validation {
  bool valid = true;
  double rms_max_abs_error = 0, rms_max_rel_error = 0;
  double softmax_max_abs_error = 0, softmax_max_rel_error = 0;
  double product_max_ratio = 0;     // max |p - ref| / tol
  double product_max_rel_error = 0; // max |p - ref| / max(|ref|, sum |terms| * 2^-24)
  // Block-scaled variants only: max |p - ref_bf16| / sum |terms| against the
  // bf16-activation reference (the error activation quantization adds).
  double product_bf16_act_rel_error = 0;
  ProductCheck product;
};

struct Outputs {
  const float *normalized;  // batch x size
  const float *softmax;     // batch x size
  const float *product;     // rows, or batch x rows for batched variants
};

// Quantized operands as the device used them (host copies), for the
// dequantize-then-matmul oracle of the quantized variants.
struct QuantOperands {
  std::vector<uint16_t> x_bf16;   // batch x size
  std::vector<uint8_t> codes;     // mxfp4: rows x size/2; fp8: rows x size
  std::vector<uint8_t> scales_e8; // mxfp4: rows x size/32
  std::vector<float> scales_f32;  // fp8: rows
  // Block-scaled variants: the device's MXFP8 activations, row-major codes
  // [batch][size] and scale bytes [batch][size / 32].
  std::vector<uint8_t> x_codes, x_scales;
};

Validation validate_all(const Options &options, const Inputs &inputs, const Outputs &outputs,
                        const QuantOperands *quant, int threads = 0);

// ---------------------------------------------------------------------------
// Dumps. L2CDUMP1 (llama2c/llama2c_common.h:16-32) for matvec variants;
// L2CDUMP2 for batched variants: the same header plus an int32 matmul code and
// an int32 pad, then normalized, softmax, product[batch*rows],
// tolerance[batch*rows] (f32), reference[batch*rows] (f64).

struct Dump {
  std::string magic;
  int32_t batch = 0, size = 0, rows = 0, inputs = 0;
  uint64_t seed = 0;
  int32_t matmul = -1;  // -1 for L2CDUMP1
  std::vector<float> normalized, softmax, product, tolerance;
  std::vector<double> reference;
};

bool write_dump(const std::string &path, const Options &options, const Outputs &outputs,
                const ProductCheck &check);
bool read_dump(const std::string &path, Dump *dump, std::string *error);

// compare_dumps.py rules (llama2c/compare_dumps.py:26-135); prints a report to
// stdout and returns true when every other dump matches the reference dump.
bool compare_dumps(const std::vector<std::string> &paths);

// ---------------------------------------------------------------------------
// Runner

struct KernelTiming {
  double us = 0;       // average duration of one launch, alone on its stream
  double bytes = 0;    // algorithmic bytes per launch
  double flops = 0;    // algorithmic flops per launch (products only)
};

struct RunResult {
  int warmup_iterations = 0;
  int launches = 0;
  double gpu_ms = 0, single_us = 0, wall_ms = 0, submit_us = 0;
  double graph_capture_ms = 0, graph_instantiate_ms = 0, graph_upload_ms = 0;
  double rms_waves = 0, softmax_waves = 0, matmul_waves = 0;
  double min_bytes_per_iter = 0;
  double matmul_flops_per_iter = 0;
  int kernels_per_iter = 0;
  KernelTiming rms, softmax, matmul;
  std::string device_name, arch;
  int cu_count = 0;
  std::string error;  // non-empty on a runtime error
};

// Runs the whole protocol of llama2c/llama2c_cuda_graph.cu:260-517 on the
// device and leaves the outputs in `outputs_host` (normalized, softmax,
// product). `quant` receives the quantized operands for quantized variants.
bool run(const Options &options, const Inputs &inputs, RunResult *result,
         std::vector<float> *normalized, std::vector<float> *softmax,
         std::vector<float> *product, QuantOperands *quant);

// The key=value output line (llama2c/llama2c_cuda_graph.cu:508-517) followed
// by this build's keys.
std::string result_line(const Options &options, const RunResult &result,
                        const Validation &validation);

// Whole command-line program: parse, generate, run, validate, dump, print.
// Returns the process exit code; the result line goes to *line (and stdout
// when print is true).
int harness_main(int argc, const char *const *argv, std::string *line, bool print);

int usable_threads();

}  // namespace l2c_host
