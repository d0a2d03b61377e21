// CPU validation of the harness outputs: the rules of
// llama2c/llama2c_common.h:139-319 (double reference, absolute rmsnorm
// tolerance, relative softmax tolerance, Higham-Mary probabilistic bound for
// every product element, closed forms for deterministic inputs), applied to
// the matrix-vector variants as written and to every checked (b, r) of the
// batched and quantized variants. The benchmark-configuration tolerances
// (relative 1e-5 for rmsnorm/softmax, 1e-4 sqrt(size) or 2e-3 for products)
// are measured alongside and reported; `valid` keeps the reference meaning.
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <limits>
#include <mutex>

#include "l2c_host.h"
#include "parallel.h"

namespace l2c_host {

double gamma_probabilistic(int n) {
  const double u = std::ldexp(1.0, -24);
  const double lambda = 9.0;
  return std::expm1(lambda * std::sqrt(static_cast<double>(n)) * u + n * u * u / (1.0 - u));
}

namespace {

struct Acc {
  bool valid = true;
  double rms_abs = 0, rms_rel = 0, sm_abs = 0, sm_rel = 0, ratio = 0, prel = 0, bf16 = 0;
  void merge(const Acc &o) {
    valid = valid && o.valid;
    bf16 = std::max(bf16, o.bf16);
    rms_abs = std::max(rms_abs, o.rms_abs);
    rms_rel = std::max(rms_rel, o.rms_rel);
    sm_abs = std::max(sm_abs, o.sm_abs);
    sm_rel = std::max(sm_rel, o.sm_rel);
    ratio = std::max(ratio, o.ratio);
    prel = std::max(prel, o.prel);
  }
};

// Records a NaN as an infinite error so a poisoned output cannot pass.
inline double err_or_inf(double e) { return e == e ? e : std::numeric_limits<double>::infinity(); }

// Double-precision reference for one vector of rmsnorm and softmax
// (llama2c_common.h:247-275).
void check_vector(const Inputs &in, const Outputs &out, int size, int b, Acc *acc) {
  const size_t off = static_cast<size_t>(b) * size;
  const float *x = in.input.data() + off;
  const float *p = in.probabilities.data() + off;
  double square_sum = 0.0;
  for (int j = 0; j < size; ++j) square_sum += static_cast<double>(x[j]) * x[j];
  const double scale = 1.0 / std::sqrt(square_sum / size + static_cast<double>(kRmsEpsilon));
  double maximum = -DBL_MAX;
  for (int j = 0; j < size; ++j) maximum = std::fmax(maximum, static_cast<double>(p[j]));
  double exp_sum = 0.0;
  for (int j = 0; j < size; ++j) exp_sum += std::exp(p[j] - maximum);
  double probability_sum = 0.0;
  for (int j = 0; j < size; ++j) {
    const double expected = x[j] * scale * in.weight[j];
    const double got = out.normalized[off + j];
    const double e = err_or_inf(std::fabs(got - expected));
    if (!(std::fabs(got - expected) <= 3.0e-4)) acc->valid = false;
    acc->rms_abs = std::max(acc->rms_abs, e);
    if (expected != 0.0) acc->rms_rel = std::max(acc->rms_rel, e / std::fabs(expected));
    else acc->rms_rel = std::max(acc->rms_rel, e);
    const double ep = std::exp(p[j] - maximum) / exp_sum;
    const double actual = out.softmax[off + j];
    const double es = err_or_inf(std::fabs(actual - ep));
    if (!(std::fabs(actual - ep) <= 1.0e-9 + 1.0e-3 * ep)) acc->valid = false;
    if (!std::isfinite(actual) || actual < 0.0) acc->valid = false;
    acc->sm_abs = std::max(acc->sm_abs, es);
    if (ep > 0.0) acc->sm_rel = std::max(acc->sm_rel, es / ep);
    probability_sum += actual;
  }
  if (!(std::isfinite(probability_sum) && std::fabs(probability_sum - 1.0) <= 3.0e-4))
    acc->valid = false;
}

// The original closed-form oracle for deterministic inputs
// (llama2c_common.h:150-198), in its float arithmetic.
void check_vector_deterministic(const Inputs &in, const Outputs &out, int size, int b, Acc *acc) {
  const size_t off = static_cast<size_t>(b) * size;
  const float *x = in.input.data() + off;
  double square_sum = 0.0;
  for (int j = 0; j < size; ++j) square_sum += static_cast<double>(x[j]) * x[j];
  const float scale = 1.0f / std::sqrt(static_cast<float>(square_sum / size) + kRmsEpsilon);
  float maximum = -FLT_MAX;
  for (int j = 0; j < size; ++j) maximum = std::fmax(maximum, x[j]);
  double exp_sum = 0.0;
  for (int j = 0; j < size; ++j) exp_sum += std::exp(static_cast<double>(x[j] - maximum));
  double probability_sum = 0.0;
  for (int j = 0; j < size; ++j) {
    const float expected = x[j] * scale * in.weight[j];
    if (!(std::fabs(out.normalized[off + j] - expected) <= 3.0e-4f)) acc->valid = false;
    const float ep = static_cast<float>(std::exp(static_cast<double>(x[j] - maximum)) / exp_sum);
    if (!(std::fabs(out.softmax[off + j] - ep) <= 1.0e-9f + 1.0e-3f * std::fabs(ep)))
      acc->valid = false;
    probability_sum += out.softmax[off + j];
  }
  if (!(std::isfinite(probability_sum) && std::fabs(probability_sum - 1.0) <= 3.0e-4))
    acc->valid = false;
  for (int j = 0; j < size; ++j)
    if (!std::isfinite(out.softmax[off + j]) || out.softmax[off + j] <= 0.0f) acc->valid = false;
}

// Dequantized weight row (fp32, as the oracle's "dequantize then fp32
// matmul" uses it).
void dequant_row(const Options &o, const QuantOperands &q, int r, float *w) {
  const int size = o.size;
  if (matmul_is_mxfp4(o.matmul)) {
    const uint8_t *codes = q.codes.data() + static_cast<size_t>(r) * (size / 2);
    const uint8_t *sc = q.scales_e8.data() + static_cast<size_t>(r) * (size / 32);
    for (int k = 0; k < size; ++k) {
      const unsigned code = (codes[k / 2] >> (4 * (k % 2))) & 15u;
      w[k] = e2m1_value(code) * std::ldexp(1.0f, static_cast<int>(sc[k / 32]) - 127);
    }
  } else {
    const uint8_t *codes = q.codes.data() + static_cast<size_t>(r) * size;
    const float s = q.scales_f32[r];
    for (int k = 0; k < size; ++k) w[k] = e4m3_value(codes[k]) * s;
  }
}

}  // namespace

Validation validate_all(const Options &o, const Inputs &in, const Outputs &out,
                        const QuantOperands *quant, int threads) {
  if (threads <= 0) threads = usable_threads();
  const bool deterministic = o.inputs.mode == InputMode::kDeterministic;
  const int batch = o.batch, size = o.size, rows = o.rows;
  Validation v;
  std::mutex lock;
  Acc total;

  // rmsnorm and softmax: every vector.
  parallel_ranges(static_cast<size_t>(batch), threads, [&](size_t b0, size_t b1, size_t) {
    Acc acc;
    for (size_t b = b0; b < b1; ++b) {
      check_vector(in, out, size, static_cast<int>(b), &acc);
      if (deterministic) check_vector_deterministic(in, out, size, static_cast<int>(b), &acc);
    }
    std::lock_guard<std::mutex> g(lock);
    total.merge(acc);
  });

  const double gamma = gamma_probabilistic(size);
  const bool batched = matmul_is_batched(o.matmul);
  const bool quantized = matmul_is_quantized(o.matmul);
  ProductCheck &pc = v.product;

  // Which vectors of the batch multiply the matrix: vector 0 for the
  // matrix-vector variants; all, or an even sample of up to 8 including both
  // ends (as applications/loom_private/decoder/oracle.cpp:97-102 samples), for
  // batched variants.
  std::vector<int> sampled;
  if (!batched) {
    sampled.push_back(0);
  } else {
    const double work = static_cast<double>(batch) * rows * size;
    if (o.full_check || work <= 8.0e9) {
      for (int b = 0; b < batch; ++b) sampled.push_back(b);
    } else {
      const int count = std::min(8, batch);
      for (int i = 0; i < count; ++i) {
        const int b = count == 1 ? 0 : static_cast<int>(static_cast<long long>(i) * (batch - 1) / (count - 1));
        if (sampled.empty() || sampled.back() != b) sampled.push_back(b);
      }
    }
    pc.sampled_batch_rows = sampled;
  }
  const size_t out_elems = batched ? static_cast<size_t>(batch) * rows : static_cast<size_t>(rows);
  pc.tolerance.assign(out_elems, batched ? std::numeric_limits<float>::quiet_NaN() : 0.0f);
  pc.reference.assign(out_elems, batched ? std::numeric_limits<double>::quiet_NaN() : 0.0);

  // Activations as the product saw them (bf16-rounded for quantized variants;
  // for the block-scaled ones, the device's MXFP8 codes times their block
  // scales, exact in float).
  std::vector<float> xq, x16;
  const bool scaled = matmul_is_scaled(o.matmul);
  if (quantized) {
    xq.resize(static_cast<size_t>(batch) * size);
    for (size_t i = 0; i < xq.size(); ++i) xq[i] = bf16_value(quant->x_bf16[i]);
  }
  if (scaled) {
    x16.swap(xq);
    xq.resize(x16.size());
    for (size_t i = 0; i < xq.size(); ++i)
      xq[i] = std::ldexp(e4m3_value(quant->x_codes[i]), static_cast<int>(quant->x_scales[i / 32]) - 127);
  }
  const float *xs = quantized ? xq.data() : in.input.data();
  // The block-scaled products take the implementation-check bound of a
  // block-scaled GEMM, experiments/blackwell/lowprec/spec.json:55-62:
  // gamma_K sum |terms| + u |reference| with u = 2^-23.
  const double u23 = std::ldexp(1.0, -23);
  const double gamma_k = static_cast<double>(size) * u23 / (1.0 - static_cast<double>(size) * u23);

  parallel_ranges(static_cast<size_t>(rows), threads, [&](size_t r0, size_t r1, size_t) {
    Acc acc;
    std::vector<float> wrow(quantized ? size : 0);
    for (size_t r = r0; r < r1; ++r) {
      const float *m = in.matrix.data() + r * size;
      if (quantized) {
        dequant_row(o, *quant, static_cast<int>(r), wrow.data());
        m = wrow.data();
      }
      for (int b : sampled) {
        const float *x = xs + static_cast<size_t>(b) * size;
        double sum = 0.0, magnitude = 0.0;
        for (int c = 0; c < size; ++c) {
          const double term = static_cast<double>(m[c]) * x[c];
          sum += term;
          magnitude += std::fabs(term);
        }
        double tolerance = gamma * magnitude + FLT_MIN;
        if (scaled) {
          tolerance = gamma_k * magnitude + u23 * std::fabs(sum) + FLT_MIN;
          // Against the bf16 activations (reported, not a validity condition).
          const float *x2 = x16.data() + static_cast<size_t>(b) * size;
          double s16 = 0.0, m16 = 0.0;
          for (int c = 0; c < size; ++c) {
            const double term = static_cast<double>(m[c]) * x2[c];
            s16 += term;
            m16 += std::fabs(term);
          }
          const double got16 = out.product[static_cast<size_t>(b) * rows + r];
          acc.bf16 = std::max(acc.bf16, err_or_inf(std::fabs(got16 - s16)) / (m16 > 0 ? m16 : 1.0));
        }
        const size_t at = batched ? static_cast<size_t>(b) * rows + r : r;
        pc.tolerance[at] = static_cast<float>(tolerance);
        pc.reference[at] = sum;
        const double got = out.product[at];
        const double e = err_or_inf(std::fabs(got - sum));
        if (!(std::fabs(got - sum) <= tolerance)) acc.valid = false;
        acc.ratio = std::max(acc.ratio, e / tolerance);
        acc.prel = std::max(acc.prel, magnitude > 0 ? e / magnitude : e);
        if (deterministic && !quantized) {
          // Closed form: the shifted identity picks input[b][r % size].
          const float expected = in.input[static_cast<size_t>(b) * size + r % static_cast<size_t>(size)];
          if (!(std::fabs(out.product[at] - expected) <= 1.0e-4f)) acc.valid = false;
          pc.tolerance[at] = std::fmin(pc.tolerance[at], 1.0e-4f);
        }
      }
    }
    std::lock_guard<std::mutex> g(lock);
    total.merge(acc);
  });

  v.valid = total.valid;
  v.rms_max_abs_error = total.rms_abs;
  v.rms_max_rel_error = total.rms_rel;
  v.softmax_max_abs_error = total.sm_abs;
  v.softmax_max_rel_error = total.sm_rel;
  v.product_max_ratio = total.ratio;
  v.product_max_rel_error = total.prel;
  v.product_bf16_act_rel_error = total.bf16;
  return v;
}

}  // namespace l2c_host
