// Command line, input generation and the quantized-format encoders of the
// llama2c harness.
#include <sched.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <thread>

#include "l2c_host.h"
#include "parallel.h"

namespace l2c_host {

const char *matmul_name(Matmul m) {
  switch (m) {
    case Matmul::kNaive: return "naive";
    case Matmul::kCoalesced: return "coalesced";
    case Matmul::kFused: return "fused";
    case Matmul::kBatched: return "batched";
    case Matmul::kMxfp4: return "mxfp4";
    case Matmul::kFp8: return "fp8";
    case Matmul::kMxfp4s: return "mxfp4s";
    case Matmul::kFp8s: return "fp8s";
  }
  return "?";
}

const char *input_name(InputMode m) {
  switch (m) {
    case InputMode::kDeterministic: return "deterministic";
    case InputMode::kRandom: return "random";
    case InputMode::kScaled: return "scaled";
    case InputMode::kNormal: return "normal";
  }
  return "?";
}

int usable_threads() {
  cpu_set_t set;
  CPU_ZERO(&set);
  if (sched_getaffinity(0, sizeof(set), &set) == 0) {
    const int n = CPU_COUNT(&set);
    if (n > 0) return n;
  }
  const unsigned n = std::thread::hardware_concurrency();
  return n > 0 ? static_cast<int>(n) : 1;
}

// ---------------------------------------------------------------------------
// Command line (llama2c/llama2c_cuda_graph.cu:195-258, llama2c_common.h:55-88).

std::string usage_text(const char *program) {
  std::string text = "Usage: ";
  text += program;
  text +=
      " [graph|direct] [launches|auto] [batch] [size] [rows] [repeats] [warmup_ms]"
      " [copy|nocopy] [naive|coalesced|fused|batched|mxfp4|fp8|mxfp4s|fp8s]"
      " [deterministic|random[=SEED]|scaled[=SEED]|normal[=SEED]] [fullcheck] [onestream] [hostwrite]"
      " [warmup_iters=N]"
      " [--dump=FILE]\n";
  return text;
}

static bool positive_int(const char *text, int *value) {
  char *end = nullptr;
  const long parsed = std::strtol(text, &end, 10);
  if (*text == '\0' || *end != '\0' || parsed <= 0 || parsed > std::numeric_limits<int>::max())
    return false;
  *value = static_cast<int>(parsed);
  return true;
}

// Input-mode tokens; returns 1 if consumed, 0 if not an input token, -1 on a
// malformed seed.
static int parse_input_token(const char *arg, InputOptions *in, std::string *error) {
  struct Mode {
    const char *name;
    InputMode mode;
  };
  static const Mode modes[] = {{"random", InputMode::kRandom},
                               {"scaled", InputMode::kScaled},
                               {"normal", InputMode::kNormal}};
  if (std::strcmp(arg, "deterministic") == 0) {
    in->mode = InputMode::kDeterministic;
    in->seed = 0;
    return 1;
  }
  for (const Mode &m : modes) {
    const size_t n = std::strlen(m.name);
    if (std::strcmp(arg, m.name) == 0) {
      in->mode = m.mode;
      in->seed = 1;
      return 1;
    }
    if (std::strncmp(arg, m.name, n) == 0 && arg[n] == '=') {
      char *end = nullptr;
      errno = 0;
      const unsigned long long seed = std::strtoull(arg + n + 1, &end, 10);
      if (arg[n + 1] == '\0' || *end != '\0' || errno != 0) {
        if (error) *error = std::string("bad seed in '") + arg + "'";
        return -1;
      }
      in->mode = m.mode;
      in->seed = seed;
      return 1;
    }
  }
  if (std::strncmp(arg, "--dump=", 7) == 0) {
    in->dump_path = arg + 7;
    return 1;
  }
  return 0;
}

bool parse_options(int argc, const char *const *argv, Options *options, std::string *error) {
  int positional = 0;
  for (int index = 1; index < argc; ++index) {
    const char *arg = argv[index];
    const int input = parse_input_token(arg, &options->inputs, error);
    if (input < 0) return false;
    if (input > 0) continue;
    struct Word {
      const char *name;
      int kind;  // 0 graph, 1 direct, 2 nocopy, 3 copy, 4 matmul, 5 fullcheck, 6 onestream, 7 hostwrite
      Matmul matmul;
    };
    static const Word words[] = {
        {"graph", 0, Matmul::kNaive},         {"direct", 1, Matmul::kNaive},
        {"nocopy", 2, Matmul::kNaive},        {"copy", 3, Matmul::kNaive},
        {"naive", 4, Matmul::kNaive},         {"coalesced", 4, Matmul::kCoalesced},
        {"fused", 4, Matmul::kFused},         {"batched", 4, Matmul::kBatched},
        {"mxfp4", 4, Matmul::kMxfp4},         {"fp8", 4, Matmul::kFp8},
        {"mxfp4s", 4, Matmul::kMxfp4s},       {"fp8s", 4, Matmul::kFp8s},
        {"fullcheck", 5, Matmul::kNaive},     {"onestream", 6, Matmul::kNaive},
        {"hostwrite", 7, Matmul::kNaive}};
    bool matched = false;
    for (const Word &w : words) {
      if (std::strcmp(arg, w.name) != 0) continue;
      matched = true;
      switch (w.kind) {
        case 0: options->graph = true; break;
        case 1: options->graph = false; break;
        case 2: options->copy_outputs = false; break;
        case 3: options->copy_outputs = true; break;
        case 4: options->matmul = w.matmul; break;
        case 5: options->full_check = true; break;
        case 6: options->one_stream = true; break;
        case 7: options->host_write = true; break;
      }
      break;
    }
    if (matched) continue;
    if (std::strncmp(arg, "warmup_iters=", 13) == 0) {
      if (!positive_int(arg + 13, &options->warmup_iters)) return false;
      continue;
    }
    if (positional == 0 && std::strcmp(arg, "auto") == 0) {
      options->auto_launches = true;
      ++positional;
      continue;
    }
    int *destination = nullptr;
    if (positional == 0) destination = &options->launches;
    if (positional == 1) destination = &options->batch;
    if (positional == 2) destination = &options->size;
    if (positional == 3) destination = &options->rows;
    if (positional == 4) destination = &options->repeats;
    if (positional == 5) destination = &options->warmup_ms;
    if (destination == nullptr || !positive_int(arg, destination)) return false;
    ++positional;
  }
  const char *dump = std::getenv("LLAMA2C_DUMP");
  if (dump != nullptr && *dump != '\0' && options->inputs.dump_path.empty())
    options->inputs.dump_path = dump;
  return true;
}

// ---------------------------------------------------------------------------
// Generators

uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

float uniform(uint64_t seed, uint64_t stream, uint64_t index) {
  const uint64_t bits = splitmix64(splitmix64(seed * 4 + stream) ^ index);
  // Top 24 bits: an integer in [0, 2^24), then scaled to [-1, 1). Both steps
  // are exact in fp32.
  return static_cast<float>(static_cast<int64_t>(bits >> 40)) * (1.0f / 8388608.0f) - 1.0f;
}

// Draw n of splitmix64 seeded with s0 is mix(s0 + n * golden), so pair p of
// the Box-Muller sequence needs only draws 2p and 2p + 1.
float normal(uint64_t seed, uint64_t stream, uint64_t index) {
  const uint64_t s0 = seed * 0x100000001b3ull + stream;
  const uint64_t pair = index / 2;
  const uint64_t d1 = splitmix64(s0 + (2 * pair) * 0x9e3779b97f4a7c15ull);
  const uint64_t d2 = splitmix64(s0 + (2 * pair + 1) * 0x9e3779b97f4a7c15ull);
  const double u1 = static_cast<double>(d1 >> 11) * 0x1.0p-53;
  const double u2 = static_cast<double>(d2 >> 11) * 0x1.0p-53;
  const double radius = std::sqrt(-2.0 * std::log(1.0 - u1));
  const double angle = 6.283185307179586476925286766559 * u2;
  return static_cast<float>(index % 2 == 0 ? radius * std::cos(angle) : radius * std::sin(angle));
}

void fill_inputs(const InputOptions &options, int batch, int size, int rows, Inputs *inputs,
                 int threads) {
  const size_t vector_elements = static_cast<size_t>(batch) * size;
  const size_t matrix_elements = static_cast<size_t>(rows) * size;
  inputs->input.assign(vector_elements, 0.0f);
  inputs->probabilities.assign(vector_elements, 0.0f);
  inputs->weight.assign(size, 1.0f);
  inputs->matrix.assign(matrix_elements, 0.0f);
  if (threads <= 0) threads = usable_threads();
  float *in = inputs->input.data(), *pr = inputs->probabilities.data();
  float *w = inputs->weight.data(), *m = inputs->matrix.data();
  if (options.mode == InputMode::kDeterministic) {
    parallel_for(vector_elements, threads, [&](size_t i) {
      in[i] = 1.0f + static_cast<float>(i % 4);
      pr[i] = 1.0f + static_cast<float>(i % 4);
    });
    parallel_for(static_cast<size_t>(rows), threads, [&](size_t r) {
      m[r * size + (r % static_cast<size_t>(size))] = 1.0f;
    });
    return;
  }
  const uint64_t seed = options.seed;
  parallel_for(vector_elements, threads, [&](size_t i) {
    in[i] = uniform(seed, 0, i);
    pr[i] = uniform(seed, 1, i);
  });
  if (options.mode == InputMode::kRandom) {
    for (int i = 0; i < size; ++i) w[i] = uniform(seed, 2, i);
    parallel_for(matrix_elements, threads, [&](size_t i) { m[i] = uniform(seed, 3, i); });
    return;
  }
  for (int i = 0; i < size; ++i) w[i] = 1.0f + 0.5f * uniform(seed, 2, i);
  const float inv_sqrt = static_cast<float>(1.0 / std::sqrt(static_cast<double>(size)));
  if (options.mode == InputMode::kScaled)
    parallel_for(matrix_elements, threads, [&](size_t i) { m[i] = uniform(seed, 3, i) * inv_sqrt; });
  else
    parallel_for(matrix_elements, threads, [&](size_t i) { m[i] = normal(seed, 3, i) * inv_sqrt; });
}

// ---------------------------------------------------------------------------
// Format encoders. The element and scale rules follow
// experiments/blackwell/lowprec/spec.json:20-27 (nearest, ties to the code
// whose least significant magnitude bit is 0, saturation, -0 -> +0) and
// reference.cpp:84-96 (bf16).

uint16_t bf16_bits(float v) {
  uint32_t bits;
  std::memcpy(&bits, &v, 4);
  if ((bits & 0x7f800000u) == 0x7f800000u) return static_cast<uint16_t>(bits >> 16);  // inf/nan
  const uint32_t lsb = (bits >> 16) & 1u;
  uint32_t r = (bits + 0x7fffu + lsb) >> 16;
  if ((r & 0x7fffu) == 0x7f80u) --r;  // finite values stay finite
  return static_cast<uint16_t>(r);
}

float bf16_value(uint16_t b) {
  const uint32_t bits = static_cast<uint32_t>(b) << 16;
  float v;
  std::memcpy(&v, &bits, 4);
  return v;
}

float e2m1_value(unsigned code) {
  static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  const float v = mag[code & 7u];
  return (code & 8u) ? -v : v;
}

// Nearest magnitude code among `count` increasing magnitudes; ties go to the
// even code; values above the last magnitude saturate to it.
static unsigned nearest_code(const double *mags, unsigned count, double a) {
  unsigned lo = 0, hi = count - 1;
  if (a >= mags[hi]) return hi;
  // Largest code with mags[code] <= a.
  while (lo < hi) {
    const unsigned mid = (lo + hi + 1) / 2;
    if (mags[mid] <= a) lo = mid;
    else hi = mid - 1;
  }
  if (mags[lo] == a) return lo;
  const double down = a - mags[lo], up = mags[lo + 1] - a;
  if (up < down) return lo + 1;
  if (down < up) return lo;
  return (lo % 2 == 0) ? lo : lo + 1;
}

unsigned e2m1_encode(double v) {
  static const double mags[8] = {0, 0.5, 1, 1.5, 2, 3, 4, 6};
  const unsigned code = nearest_code(mags, 8, std::fabs(v));
  return (code != 0 && v < 0) ? (code | 8u) : code;
}

float e4m3_value(unsigned code) {
  const unsigned e = (code >> 3) & 15u, m = code & 7u;
  const float mag = e == 0 ? std::ldexp(static_cast<float>(m) / 8.0f, -6)
                           : std::ldexp(1.0f + static_cast<float>(m) / 8.0f, static_cast<int>(e) - 7);
  return (code & 0x80u) ? -mag : mag;
}

unsigned e4m3_encode(float v) {
  // A function-local static is initialized once, thread-safely: the encoder
  // may be called from the validation's worker threads.
  struct Table {
    double mags[127];
    Table() {
      for (unsigned c = 0; c < 127; ++c) mags[c] = e4m3_value(c);
    }
  };
  static const Table table;
  const unsigned code = nearest_code(table.mags, 127, std::fabs(static_cast<double>(v)));
  return (code != 0 && v < 0) ? (code | 0x80u) : code;
}

int mxfp4_block_exponent(float amax) {
  if (!(amax > 0.0f)) return -127;
  // Largest X with 6 * 2^X <= amax: with amax = m * 2^E, m in [1, 2),
  // 6 * 2^X = 1.5 * 2^(X + 2), so X = E - 2 when m >= 1.5 and E - 3 otherwise.
  const int e = std::ilogb(amax);
  const double m = std::ldexp(static_cast<double>(amax), -e);
  const int x = m >= 1.5 ? e - 2 : e - 3;
  return std::min(127, std::max(-127, x));
}

int mxfp8_block_exponent(float amax) {
  if (!(amax > 0.0f)) return -127;
  // Smallest X with amax <= 448 * 2^X = 1.75 * 2^(X + 8): with amax = m * 2^E,
  // m in [1, 2), X = E - 8 when m <= 1.75 and E - 7 otherwise.
  const int e = std::ilogb(amax);
  const double m = std::ldexp(static_cast<double>(amax), -e);
  const int x = m <= 1.75 ? e - 8 : e - 7;
  return std::min(127, std::max(-127, x));
}

}  // namespace l2c_host
