// Device kernels of the batched greedy decoder (rmsnorm of each sequence's
// current token -> dense classifier -> softmax + argmax with the argmax fed
// back as the next token), the pipeline of
// applications/loom_private/decoder/decoder.cu:200-367. The classifier itself
// is l2c_matmul (gemm_f32_mfma_kernel); this file holds the model generator
// and the two row kernels around it.
//
// Row kernels: one workgroup of 256 lanes per sequence. Rows up to 16384
// values are register-resident: each lane loads its slice once (16-byte
// loads where the row is 16-byte aligned), the reductions run on registers,
// and the result is written once, so a row costs one read and one write of
// HBM. Longer rows stream through the same lanes in passes. Reductions are
// wave64 butterflies combined across the four waves in wave order, so every
// result is deterministic (the decoder's check compares repeated
// invocations and direct against graph launches bitwise).
#include <climits>

#include "l2c_common.h"
#include "../../include/l2c.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / L2C_WAVE;

// Synthetic model (decoder.cu:30-43): embedding row t is 1 except 4 at
// column t; the norm weight is 1; classifier row r is 0 except 1 at column
// (r + vocab - 1) mod vocab.
__global__ void decoder_init_model_kernel(float *embedding, float *classifier, float *norm_weight,
                                          int width, int vocab) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  const size_t first = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t total = static_cast<size_t>(vocab) * width;
  for (size_t i = first; i < total; i += stride) {
    const int row = static_cast<int>(i / width);
    const int column = static_cast<int>(i % width);
    embedding[i] = column == row ? 4.0f : 1.0f;
    classifier[i] = column == (row + vocab - 1) % vocab ? 1.0f : 0.0f;
  }
  for (size_t j = first; j < static_cast<size_t>(width); j += stride) norm_weight[j] = 1.0f;
}

// Sum over the workgroup: butterflies within each wave, then the four wave
// totals in wave order. `slots` holds kWaves floats; callers alternate slot
// sets between consecutive reductions.
__device__ __forceinline__ float group_sum(float v, float *slots) {
  v = l2c::wave_sum(v);
  if (threadIdx.x % L2C_WAVE == 0) slots[threadIdx.x / L2C_WAVE] = v;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) total += slots[w];
  return total;
}

__device__ __forceinline__ float group_max(float v, float *slots) {
  v = l2c::wave_max(v);
  if (threadIdx.x % L2C_WAVE == 0) slots[threadIdx.x / L2C_WAVE] = v;
  __syncthreads();
  float m = slots[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) m = fmaxf(m, slots[w]);
  return m;
}

// The workgroup's maximum of |normalized| (NaNs ignored, as fmaxf does) into
// the word at `absmax` as float bits: non-negative floats order as their bit
// patterns, so an unsigned atomic maximum is the float maximum, exactly and
// in any order.
__device__ __forceinline__ void publish_absmax(float m, float *mslots, unsigned *absmax) {
  m = group_max(m, mslots);
  if (threadIdx.x == 0) atomicMax(absmax, __float_as_uint(m));
}

// llama2.c rmsnorm of the embedding row of each sequence's current token
// (decoder.cu:45-77): ss = sum x^2; ss /= width; ss += 1e-5f;
// scale = 1 / sqrtf(ss); o_j = w_j * (scale * x_j). An out-of-range token
// (a corrupted state, or the poisoned token buffer) gives a NaN row, so the
// check fails instead of reading outside the embedding.
template <bool VEC, bool AMAX>
__global__ __launch_bounds__(kThreads) void decoder_rmsnorm_kernel(float *normalized,
                                                                   const int *tokens,
                                                                   const float *embedding,
                                                                   const float *weight, int width,
                                                                   int vocab, unsigned *absmax) {
#pragma clang fp contract(off)  // separate multiply and add, as the contract's builds
  __shared__ float slots[kWaves];
  __shared__ float mslots[kWaves];
  const int sequence = blockIdx.x;
  const int token = tokens[sequence];
  float *o = normalized + static_cast<size_t>(sequence) * width;
  const int t = threadIdx.x;
  if (token < 0 || token >= vocab) {
    for (int j = t; j < width; j += kThreads) o[j] = __builtin_nanf("");
    return;
  }
  const float *x = embedding + static_cast<size_t>(token) * width;
  float ss = 0.0f;
  if constexpr (VEC) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    for (int c = t; c < width / 4; c += kThreads) {
      const float4 v = x4[c];
      ss += v.x * v.x;
      ss += v.y * v.y;
      ss += v.z * v.z;
      ss += v.w * v.w;
    }
  } else {
    for (int j = t; j < width; j += kThreads) ss += x[j] * x[j];
  }
  ss = group_sum(ss, slots);
  ss /= static_cast<float>(width);
  ss += 1e-5f;
  const float scale = 1.0f / sqrtf(ss);
  float m = 0.0f;
  if constexpr (VEC) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const float4 *w4 = reinterpret_cast<const float4 *>(weight);
    float4 *o4 = reinterpret_cast<float4 *>(o);
    for (int c = t; c < width / 4; c += kThreads) {
      const float4 v = x4[c], g = w4[c];
      const float4 y = make_float4(g.x * (scale * v.x), g.y * (scale * v.y), g.z * (scale * v.z),
                                   g.w * (scale * v.w));
      o4[c] = y;
      if constexpr (AMAX) m = fmaxf(m, fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w))));
    }
  } else {
    for (int j = t; j < width; j += kThreads) {
      const float y = weight[j] * (scale * x[j]);
      o[j] = y;
      if constexpr (AMAX) m = fmaxf(m, fabsf(y));
    }
  }
  if constexpr (AMAX) publish_absmax(m, mslots, absmax);
}

// Register-resident rmsnorm: lane t holds float4 chunks t + 256 c (VEC) or
// values t + 256 i of the row, c < CHUNKS (4 * CHUNKS values a lane).
template <int CHUNKS, bool VEC, bool AMAX>
__global__ __launch_bounds__(kThreads) void decoder_rmsnorm_regs_kernel(float *normalized, const int *tokens,
                                                                        const float *embedding,
                                                                        const float *weight, int width,
                                                                        int vocab, unsigned *absmax) {
#pragma clang fp contract(off)
  __shared__ float slots[kWaves];
  __shared__ float mslots[kWaves];
  const int sequence = blockIdx.x;
  const int token = tokens[sequence];
  float *o = normalized + static_cast<size_t>(sequence) * width;
  const int t = threadIdx.x;
  if (token < 0 || token >= vocab) {
    for (int j = t; j < width; j += kThreads) o[j] = __builtin_nanf("");
    return;
  }
  const float *x = embedding + static_cast<size_t>(token) * width;
  float v[4 * CHUNKS];
  if constexpr (VEC) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int i = t + c * kThreads;
      const float4 q = i < width / 4 ? x4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      v[4 * c] = q.x, v[4 * c + 1] = q.y, v[4 * c + 2] = q.z, v[4 * c + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4 * CHUNKS; ++i) {
      const int j = t + i * kThreads;
      v[i] = j < width ? x[j] : 0.0f;
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 4 * CHUNKS; ++i) ss += v[i] * v[i];
  ss = group_sum(ss, slots);
  ss /= static_cast<float>(width);
  ss += 1e-5f;
  const float scale = 1.0f / sqrtf(ss);
  float m = 0.0f;
  if constexpr (VEC) {
    const float4 *w4 = reinterpret_cast<const float4 *>(weight);
    float4 *o4 = reinterpret_cast<float4 *>(o);
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int i = t + c * kThreads;
      if (i < width / 4) {
        const float4 g = w4[i];
        const float4 y = make_float4(g.x * (scale * v[4 * c]), g.y * (scale * v[4 * c + 1]),
                                     g.z * (scale * v[4 * c + 2]), g.w * (scale * v[4 * c + 3]));
        o4[i] = y;
        if constexpr (AMAX) m = fmaxf(m, fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w))));
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4 * CHUNKS; ++i) {
      const int j = t + i * kThreads;
      if (j < width) {
        const float y = weight[j] * (scale * v[i]);
        o[j] = y;
        if constexpr (AMAX) m = fmaxf(m, fabsf(y));
      }
    }
  }
  if constexpr (AMAX) publish_absmax(m, mslots, absmax);
}

// The VEC register-resident rmsnorm over ROWS consecutive sequences per
// workgroup, software-pipelined: row r + 1's loads are issued before row r is
// reduced and stored, so reads and writes overlap inside a CU instead of the
// whole grid reading, then writing. The norm weight is loaded once. Per row the
// arithmetic, and its order, are those of decoder_rmsnorm_regs_kernel.
template <int CHUNKS>
__device__ __forceinline__ void rms_row_load(float4 (&dst)[CHUNKS], const float *embedding, int token, int vocab,
                                             int width, int t) {
  const bool ok = token >= 0 && token < vocab;
  const float4 *x4 = reinterpret_cast<const float4 *>(embedding + static_cast<size_t>(ok ? token : 0) * width);
  const int n4 = width / 4;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c)
    dst[c] = ok && t + c * kThreads < n4 ? x4[t + c * kThreads] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

template <int CHUNKS, bool AMAX>
__device__ __forceinline__ void rms_row_store(float *o, const float4 (&v)[CHUNKS], const float4 (&g)[CHUNKS],
                                              bool ok, float *slots, int width, int t, float &m) {
#pragma clang fp contract(off)
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    ss += v[c].x * v[c].x;
    ss += v[c].y * v[c].y;
    ss += v[c].z * v[c].z;
    ss += v[c].w * v[c].w;
  }
  ss = group_sum(ss, slots);
  ss /= static_cast<float>(width);
  ss += 1e-5f;
  const float scale = 1.0f / sqrtf(ss);
  float4 *o4 = reinterpret_cast<float4 *>(o);
  const int n4 = width / 4;
  const float nan = __builtin_nanf("");
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int i = t + c * kThreads;
    if (i < n4) {
      const float4 y = ok ? make_float4(g[c].x * (scale * v[c].x), g[c].y * (scale * v[c].y),
                                        g[c].z * (scale * v[c].z), g[c].w * (scale * v[c].w))
                          : make_float4(nan, nan, nan, nan);
      o4[i] = y;
      if constexpr (AMAX) m = fmaxf(m, fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w))));
    }
  }
}

// Two rows a workgroup (221 VGPRs, two workgroups a CU) against one row a
// workgroup at 1024 x 16384, same box: 24.5 against 26.4 µs in the decoder,
// 24.0 / 28.2 / 26.7 against 26.3 / 29.3 / 27.8 µs in the lowprec fp32 / bf16 /
// NVFP4 steps, 27.9 against 26.9 µs in the MXFP6 step; four rows (one
// workgroup a CU) measured 28.7 µs. Used from this batch up, where the grid
// still gives every CU two workgroups.
constexpr int kRowsPipelineMinBatch = 512;

template <int CHUNKS, int ROWS, bool AMAX>
__global__ __launch_bounds__(kThreads) void decoder_rmsnorm_rows_kernel(float *normalized, const int *tokens,
                                                                        const float *embedding,
                                                                        const float *weight, int width,
                                                                        int vocab, int batch, unsigned *absmax) {
  static_assert(ROWS % 2 == 0, "rows alternate between two register sets");
  __shared__ float slots[2][kWaves];
  __shared__ float mslots[kWaves];
  float m = 0.0f;
  const int t = threadIdx.x;
  const int first = blockIdx.x * ROWS;
  float4 g[CHUNKS], a[CHUNKS], b[CHUNKS];
  const float4 *w4 = reinterpret_cast<const float4 *>(weight);
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c)
    g[c] = t + c * kThreads < width / 4 ? w4[t + c * kThreads] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  int token_a = tokens[first];  // first < batch: the grid is ceil(batch / ROWS)
  rms_row_load(a, embedding, token_a, vocab, width, t);
#pragma unroll
  for (int r = 0; r < ROWS; r += 2) {
    // Row first + r is in a; first + r + 1 goes to b.
    const bool has_b = first + r + 1 < batch;
    const int token_b = has_b ? tokens[first + r + 1] : -1;
    if (has_b) rms_row_load(b, embedding, token_b, vocab, width, t);
    rms_row_store<CHUNKS, AMAX>(normalized + static_cast<size_t>(first + r) * width, a, g,
                                token_a >= 0 && token_a < vocab, slots[0], width, t, m);
    if (!has_b) break;  // uniform across the workgroup
    const bool has_a = r + 2 < ROWS && first + r + 2 < batch;
    if (has_a) {
      token_a = tokens[first + r + 2];
      rms_row_load(a, embedding, token_a, vocab, width, t);
    }
    rms_row_store<CHUNKS, AMAX>(normalized + static_cast<size_t>(first + r + 1) * width, b, g,
                                token_b >= 0 && token_b < vocab, slots[1], width, t, m);
    if (!has_a) break;
  }
  if constexpr (AMAX) publish_absmax(m, mslots, absmax);
}

// (value, index) maximum over the workgroup with ties to the smaller index;
// the result is valid in lane 0. INT_MAX marks "no candidate".
__device__ __forceinline__ int group_argmax(float best, int best_index, float *vslots, int *islots) {
#pragma unroll
  for (int offset = L2C_WAVE / 2; offset > 0; offset >>= 1) {
    const float ov = __shfl_xor(best, offset, L2C_WAVE);
    const int oi = __shfl_xor(best_index, offset, L2C_WAVE);
    if (ov > best || (ov == best && oi < best_index)) {
      best = ov;
      best_index = oi;
    }
  }
  const int t = threadIdx.x;
  if (t % L2C_WAVE == 0) {
    vslots[t / L2C_WAVE] = best;
    islots[t / L2C_WAVE] = best_index;
  }
  __syncthreads();
  float v = vslots[0];
  int i = islots[0];
  for (int w = 1; w < kWaves; ++w) {
    if (vslots[w] > v || (vslots[w] == v && islots[w] < i)) {
      v = vslots[w];
      i = islots[w];
    }
  }
  return i;
}

// Register-resident softmax + argmax (same arithmetic as the streaming kernel
// below): lane t holds chunks t + 256 c (VEC) or values t + 256 i, in
// increasing index order, so a lane's first maximum is its smallest index.
template <int CHUNKS, bool VEC>
__global__ __launch_bounds__(kThreads) void decoder_softmax_argmax_regs_kernel(
    float *probabilities, const float *logits, int *tokens, int *generated, int vocab, int steps, int step) {
#pragma clang fp contract(off)
  __shared__ float slots[3 * kWaves];
  __shared__ int islots[kWaves];
  const int sequence = blockIdx.x;
  const float *x = logits + static_cast<size_t>(sequence) * vocab;
  float *p = probabilities + static_cast<size_t>(sequence) * vocab;
  const int t = threadIdx.x;
  float v[4 * CHUNKS];
  bool live[4 * CHUNKS];
  if constexpr (VEC) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int i = t + c * kThreads;
      const bool ok = i < vocab / 4;
      const float4 q = ok ? x4[i] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      v[4 * c] = q.x, v[4 * c + 1] = q.y, v[4 * c + 2] = q.z, v[4 * c + 3] = q.w;
      live[4 * c] = live[4 * c + 1] = live[4 * c + 2] = live[4 * c + 3] = ok;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4 * CHUNKS; ++i) {
      const int r = t + i * kThreads;
      live[i] = r < vocab;
      v[i] = live[i] ? x[r] : -INFINITY;
    }
  }
  float maximum = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4 * CHUNKS; ++i) maximum = fmaxf(maximum, v[i]);
  maximum = group_max(maximum, slots);
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4 * CHUNKS; ++i) {
    v[i] = live[i] ? expf(v[i] - maximum) : 0.0f;
    sum += v[i];
  }
  sum = group_sum(sum, slots + kWaves);
  float best = -INFINITY;
  int best_index = INT_MAX;
#pragma unroll
  for (int i = 0; i < 4 * CHUNKS; ++i) {
    const float q = v[i] / sum;
    v[i] = q;
    const int index = VEC ? 4 * (t + (i / 4) * kThreads) + i % 4 : t + i * kThreads;
    if (live[i] && q > best) {
      best = q;
      best_index = index;
    }
  }
  if constexpr (VEC) {
    float4 *p4 = reinterpret_cast<float4 *>(p);
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int i = t + c * kThreads;
      if (i < vocab / 4) p4[i] = make_float4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4 * CHUNKS; ++i) {
      const int r = t + i * kThreads;
      if (r < vocab) p[r] = v[i];
    }
  }
  const int i = group_argmax(best, best_index, slots + 2 * kWaves, islots);
  if (t == 0) {
    const int next = i == INT_MAX ? -1 : i;
    tokens[sequence] = next;
    generated[static_cast<size_t>(sequence) * steps + step] = next;
  }
}

// llama2.c softmax (max-subtracted expf divided by the float sum) followed by
// sample_argmax (the first maximum of the probabilities), decoder.cu:127-198.
// The argmax is the sequence's next token: written to tokens[sequence] for
// the next step and recorded in generated[sequence][step]. No maximum (every
// probability NaN) gives token -1.
__global__ __launch_bounds__(kThreads) void decoder_softmax_argmax_kernel(
    float *probabilities, const float *logits, int *tokens, int *generated, int vocab, int steps,
    int step) {
#pragma clang fp contract(off)
  __shared__ float slots[3 * kWaves];
  __shared__ int islots[kWaves];
  const int sequence = blockIdx.x;
  const float *x = logits + static_cast<size_t>(sequence) * vocab;
  float *p = probabilities + static_cast<size_t>(sequence) * vocab;
  const int t = threadIdx.x;

  float maximum = -INFINITY;
  for (int r = t; r < vocab; r += kThreads) maximum = fmaxf(maximum, x[r]);
  maximum = group_max(maximum, slots);

  float sum = 0.0f;
  for (int r = t; r < vocab; r += kThreads) {
    const float e = expf(x[r] - maximum);
    p[r] = e;
    sum += e;
  }
  sum = group_sum(sum, slots + kWaves);

  // Each lane normalizes the entries it wrote (its own stores, visible to
  // itself) and keeps the first maximum among them.
  float best = -INFINITY;
  int best_index = INT_MAX;
  for (int r = t; r < vocab; r += kThreads) {
    const float q = p[r] / sum;
    p[r] = q;
    if (q > best) {
      best = q;
      best_index = r;
    }
  }
  // (value, index) maximum with ties to the smaller index: butterflies, then
  // the waves in order.
#pragma unroll
  for (int offset = L2C_WAVE / 2; offset > 0; offset >>= 1) {
    const float ov = __shfl_xor(best, offset, L2C_WAVE);
    const int oi = __shfl_xor(best_index, offset, L2C_WAVE);
    if (ov > best || (ov == best && oi < best_index)) {
      best = ov;
      best_index = oi;
    }
  }
  float *vslots = slots + 2 * kWaves;
  if (t % L2C_WAVE == 0) {
    vslots[t / L2C_WAVE] = best;
    islots[t / L2C_WAVE] = best_index;
  }
  __syncthreads();
  if (t == 0) {
    float v = vslots[0];
    int i = islots[0];
    for (int w = 1; w < kWaves; ++w) {
      if (vslots[w] > v || (vslots[w] == v && islots[w] < i)) {
        v = vslots[w];
        i = islots[w];
      }
    }
    const int next = i == INT_MAX ? -1 : i;
    tokens[sequence] = next;
    generated[static_cast<size_t>(sequence) * steps + step] = next;
  }
}

}  // namespace

extern "C" int l2c_decoder_init_model(float *embedding, float *classifier, float *norm_weight,
                                      int width, int vocab, hipStream_t stream) {
  if (width <= 0 || vocab <= 0) return hipErrorInvalidValue;
  if (!embedding || !classifier || !norm_weight) return hipErrorInvalidValue;
  hipLaunchKernelGGL(decoder_init_model_kernel, dim3(4096), dim3(256), 0, stream, embedding,
                     classifier, norm_weight, width, vocab);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

namespace {

// The smallest register-resident instance whose lanes hold n values, or
// null for rows longer than 16384 (streamed instead).
using RmsFn = void (*)(float *, const int *, const float *, const float *, int, int, unsigned *);
using SoftFn = void (*)(float *, const float *, int *, int *, int, int, int);

template <bool VEC, bool AMAX>
RmsFn rmsnorm_regs(int n) {
  const int per_lane = (n + kThreads - 1) / kThreads;
  if (per_lane <= 4) return decoder_rmsnorm_regs_kernel<1, VEC, AMAX>;
  if (per_lane <= 8) return decoder_rmsnorm_regs_kernel<2, VEC, AMAX>;
  if (per_lane <= 16) return decoder_rmsnorm_regs_kernel<4, VEC, AMAX>;
  if (per_lane <= 32) return decoder_rmsnorm_regs_kernel<8, VEC, AMAX>;
  if (per_lane <= 64) return decoder_rmsnorm_regs_kernel<16, VEC, AMAX>;
  return nullptr;
}

template <bool VEC>
SoftFn softmax_regs(int n) {
  const int per_lane = (n + kThreads - 1) / kThreads;
  if (per_lane <= 4) return decoder_softmax_argmax_regs_kernel<1, VEC>;
  if (per_lane <= 8) return decoder_softmax_argmax_regs_kernel<2, VEC>;
  if (per_lane <= 16) return decoder_softmax_argmax_regs_kernel<4, VEC>;
  if (per_lane <= 32) return decoder_softmax_argmax_regs_kernel<8, VEC>;
  if (per_lane <= 64) return decoder_softmax_argmax_regs_kernel<16, VEC>;
  return nullptr;
}

template <bool AMAX>
int launch_decoder_rmsnorm(float *normalized, const int *tokens, const float *embedding, const float *weight,
                           int width, int vocab, int batch, unsigned *absmax, hipStream_t stream) {
  const bool vec = width % 4 == 0 && l2c_aligned16(normalized) && l2c_aligned16(embedding) &&
                   l2c_aligned16(weight);
  const int per_lane = (width + kThreads - 1) / kThreads;
  if (vec && per_lane > 32 && per_lane <= 64 && batch >= kRowsPipelineMinBatch) {
    hipLaunchKernelGGL((decoder_rmsnorm_rows_kernel<16, 2, AMAX>), dim3((batch + 1) / 2), dim3(kThreads), 0, stream,
                       normalized, tokens, embedding, weight, width, vocab, batch, absmax);
  } else if (const RmsFn regs = vec ? rmsnorm_regs<true, AMAX>(width) : rmsnorm_regs<false, AMAX>(width)) {
    hipLaunchKernelGGL(regs, dim3(batch), dim3(kThreads), 0, stream, normalized, tokens, embedding, weight, width,
                       vocab, absmax);
  } else if (vec)
    hipLaunchKernelGGL((decoder_rmsnorm_kernel<true, AMAX>), dim3(batch), dim3(kThreads), 0, stream,
                       normalized, tokens, embedding, weight, width, vocab, absmax);
  else
    hipLaunchKernelGGL((decoder_rmsnorm_kernel<false, AMAX>), dim3(batch), dim3(kThreads), 0, stream,
                       normalized, tokens, embedding, weight, width, vocab, absmax);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

}  // namespace

extern "C" int l2c_decoder_rmsnorm(float *normalized, const int *tokens, const float *embedding,
                                   const float *weight, int width, int vocab, int batch,
                                   hipStream_t stream) {
  if (width <= 0 || vocab <= 0 || batch < 0) return hipErrorInvalidValue;
  if (batch == 0) return hipSuccess;
  if (!normalized || !tokens || !embedding || !weight) return hipErrorInvalidValue;
  return launch_decoder_rmsnorm<false>(normalized, tokens, embedding, weight, width, vocab, batch, nullptr, stream);
}

extern "C" int l2c_decoder_rmsnorm_absmax(float *normalized, const int *tokens, const float *embedding,
                                          const float *weight, int width, int vocab, int batch,
                                          unsigned *absmax_bits, hipStream_t stream) {
  if (width <= 0 || vocab <= 0 || batch < 0 || !absmax_bits) return hipErrorInvalidValue;
  if (batch == 0) return hipSuccess;
  if (!normalized || !tokens || !embedding || !weight) return hipErrorInvalidValue;
  return launch_decoder_rmsnorm<true>(normalized, tokens, embedding, weight, width, vocab, batch, absmax_bits,
                                      stream);
}

extern "C" int l2c_decoder_softmax_argmax(float *probabilities, const float *logits, int *tokens,
                                          int *generated, int vocab, int batch, int steps,
                                          int step, hipStream_t stream) {
  if (vocab <= 0 || batch < 0 || steps <= 0 || step < 0 || step >= steps)
    return hipErrorInvalidValue;
  if (batch == 0) return hipSuccess;
  if (!probabilities || !logits || !tokens || !generated) return hipErrorInvalidValue;
  const bool vec = vocab % 4 == 0 && l2c_aligned16(probabilities) && l2c_aligned16(logits);
  if (const SoftFn regs = vec ? softmax_regs<true>(vocab) : softmax_regs<false>(vocab))
    hipLaunchKernelGGL(regs, dim3(batch), dim3(kThreads), 0, stream, probabilities, logits, tokens, generated, vocab,
                       steps, step);
  else
    hipLaunchKernelGGL(decoder_softmax_argmax_kernel, dim3(batch), dim3(kThreads), 0, stream,
                       probabilities, logits, tokens, generated, vocab, steps, step);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}
