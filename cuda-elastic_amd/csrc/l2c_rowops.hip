// Row kernels of the llama2c hot path on gfx950: rmsnorm, softmax, the
// matrix-vector product (naive and coalesced) and the single-launch fused
// iteration.
//
// Design (MI355X: 256 CUs in 8 XCDs, wave64, 160 KiB LDS per CU, HBM3E):
//  * rmsnorm and softmax are one-pass: a workgroup owns one row, loads it once
//    into VGPRs with 16-byte loads (V float4 per lane), reduces it with wave64
//    shuffles plus one LDS slot per wave, and writes the result from the same
//    registers. HBM traffic is the floor: one read and one write per element
//    (the reference's rmsnorm reads twice, its softmax reads 3x and writes 2x;
//    llama2c/llama2c_cuda_graph.cu:58-115).
//  * Rows whose address is not 16-byte aligned (size % 4 != 0) keep the same
//    one-pass structure with scalar loads; rows longer than 1024 lanes x 64
//    floats take a two-pass path that re-reads the row.
//  * The coalesced matrix-vector product gives each output row to one
//    wavefront: 64 lanes x 16 B = 1 KiB contiguous per load instruction, W
//    streamed with nontemporal loads so it does not evict x from L2, several
//    independent loads in flight per lane, one wave reduction per row.
//  * The naive product keeps the reference's one-lane-per-row structure and
//    its sequential column order (one fused multiply-add per column), so its
//    result is bit-reproducible by a CPU fmaf chain.
#include "l2c_common.h"
#include "../../include/l2c.h"

namespace {

using l2c::block_max;
using l2c::block_sum;

constexpr int kMaxRowThreads = 1024;
constexpr int kGenericThreads = 256;
// The fused kernel holds a matrix row and streams x beside it, so it is
// limited to 256 lanes per row (<= 16384 floats in registers).
constexpr int kFusedThreads = 256;

// ---------------------------------------------------------------------------
// Row loaders. Thread t of a T-thread block holds chunk c = t + i*T for
// i < V: a float4 (VEC) or, for unaligned rows, four scalars at element
// t + (4i+s)*T (s < 4). Missing elements read as `fill`.

template <int V, bool VEC>
struct Row {
  float4 x[V];

  __device__ __forceinline__ void load(const float *row, int size, float fill) {
    const int T = blockDim.x, t = threadIdx.x;
    if constexpr (VEC) {
      const float4 *row4 = reinterpret_cast<const float4 *>(row);
      const int cols4 = size >> 2;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const int c = t + i * T;
        x[i] = c < cols4 ? row4[c] : make_float4(fill, fill, fill, fill);
      }
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const int j0 = t + (4 * i) * T;
        x[i].x = j0 < size ? row[j0] : fill;
        x[i].y = j0 + T < size ? row[j0 + T] : fill;
        x[i].z = j0 + 2 * T < size ? row[j0 + 2 * T] : fill;
        x[i].w = j0 + 3 * T < size ? row[j0 + 3 * T] : fill;
      }
    }
  }

  // Stores x * scale * weight[j] (weight may be null: x * scale) for every
  // valid element j, with 16-byte stores on the vector path.
  __device__ __forceinline__ void store_scaled(float *row, int size, float scale,
                                               const float *weight) const {
    const int T = blockDim.x, t = threadIdx.x;
    if constexpr (VEC) {
      float4 *row4 = reinterpret_cast<float4 *>(row);
      const float4 *w4 = reinterpret_cast<const float4 *>(weight);
      const int cols4 = size >> 2;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const int c = t + i * T;
        if (c < cols4) {
          float4 r;
          if (weight != nullptr) {
            const float4 g = w4[c];
            r.x = x[i].x * scale * g.x;
            r.y = x[i].y * scale * g.y;
            r.z = x[i].z * scale * g.z;
            r.w = x[i].w * scale * g.w;
          } else {
            r.x = x[i].x * scale;
            r.y = x[i].y * scale;
            r.z = x[i].z * scale;
            r.w = x[i].w * scale;
          }
          l2c::st4_stream(row4 + c, r);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float v[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int j = t + (4 * i + s) * T;
          if (j < size) row[j] = weight != nullptr ? v[s] * scale * weight[j] : v[s] * scale;
        }
      }
    }
  }
};

// ---------------------------------------------------------------------------
// One row of each operation, executed by a whole block. `slots` is LDS
// scratch with room for two reductions (2 x 16 floats).

template <int V, bool VEC>
__device__ __forceinline__ void rmsnorm_row(float *out, const float *in, const float *weight,
                                            int size, float eps, float *slots) {
  Row<V, VEC> r;
  r.load(in, size, 0.0f);
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    ss = fmaf(r.x[i].x, r.x[i].x, ss);
    ss = fmaf(r.x[i].y, r.x[i].y, ss);
    ss = fmaf(r.x[i].z, r.x[i].z, ss);
    ss = fmaf(r.x[i].w, r.x[i].w, ss);
  }
  ss = block_sum(ss, slots);
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(size) + eps);
  r.store_scaled(out, size, scale, weight);
}

template <int V, bool VEC>
__device__ __forceinline__ void softmax_row(float *out, const float *logits, int size,
                                            float *slots) {
  Row<V, VEC> r;
  r.load(logits, size, -FLT_MAX);
  float m = -FLT_MAX;
#pragma unroll
  for (int i = 0; i < V; ++i)
    m = fmaxf(m, fmaxf(fmaxf(r.x[i].x, r.x[i].y), fmaxf(r.x[i].z, r.x[i].w)));
  m = block_max(m, slots);
  // exp of the padding (-FLT_MAX - m) underflows to exactly 0, so padding
  // adds nothing to the sum.
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    r.x[i].x = expf(r.x[i].x - m);
    r.x[i].y = expf(r.x[i].y - m);
    r.x[i].z = expf(r.x[i].z - m);
    r.x[i].w = expf(r.x[i].w - m);
    s += (r.x[i].x + r.x[i].y) + (r.x[i].z + r.x[i].w);
  }
  s = block_sum(s, slots + 16);
  const float inv = 1.0f / s;
  r.store_scaled(out, size, inv, nullptr);
}

// Dot product of one matrix row with x, by a whole block (fused kernel). The
// matrix row is loaded first (all V loads in flight), x is read per chunk.
template <int V, bool VEC>
__device__ __forceinline__ void matvec_row_block(float *out_elem, const float *mrow,
                                                 const float *x, int size, float *slots) {
  Row<V, VEC> w;
  w.load(mrow, size, 0.0f);
  const int T = blockDim.x, t = threadIdx.x;
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    float4 v;
    if constexpr (VEC) {
      const int c = t + i * T;
      v = c < (size >> 2) ? reinterpret_cast<const float4 *>(x)[c] : make_float4(0, 0, 0, 0);
    } else {
      const int j0 = t + (4 * i) * T;
      v.x = j0 < size ? x[j0] : 0.0f;
      v.y = j0 + T < size ? x[j0 + T] : 0.0f;
      v.z = j0 + 2 * T < size ? x[j0 + 2 * T] : 0.0f;
      v.w = j0 + 3 * T < size ? x[j0 + 3 * T] : 0.0f;
    }
    acc = fmaf(w.x[i].x, v.x, acc);
    acc = fmaf(w.x[i].y, v.y, acc);
    acc = fmaf(w.x[i].z, v.z, acc);
    acc = fmaf(w.x[i].w, v.w, acc);
  }
  acc = block_sum(acc, slots);
  if (threadIdx.x == 0) *out_elem = acc;
}

// Two-pass versions for rows longer than the register-resident limit.
__device__ void rmsnorm_row_generic(float *out, const float *in, const float *weight, int size,
                                    float eps, float *slots) {
  float ss = 0.0f;
  for (int j = threadIdx.x; j < size; j += blockDim.x) ss = fmaf(in[j], in[j], ss);
  ss = block_sum(ss, slots);
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(size) + eps);
  for (int j = threadIdx.x; j < size; j += blockDim.x) out[j] = in[j] * scale * weight[j];
}

__device__ void softmax_row_generic(float *out, const float *logits, int size, float *slots) {
  float m = -FLT_MAX;
  for (int j = threadIdx.x; j < size; j += blockDim.x) m = fmaxf(m, logits[j]);
  m = block_max(m, slots);
  float s = 0.0f;
  for (int j = threadIdx.x; j < size; j += blockDim.x) s += expf(logits[j] - m);
  s = block_sum(s, slots + 16);
  const float inv = 1.0f / s;
  // Separate loops so the kernel is also correct in place (out == logits).
  for (int j = threadIdx.x; j < size; j += blockDim.x) out[j] = expf(logits[j] - m) * inv;
}

__device__ void matvec_row_block_generic(float *out_elem, const float *mrow, const float *x,
                                         int size, float *slots) {
  float acc = 0.0f;
  for (int j = threadIdx.x; j < size; j += blockDim.x) acc = fmaf(mrow[j], x[j], acc);
  acc = block_sum(acc, slots);
  if (threadIdx.x == 0) *out_elem = acc;
}

// ---------------------------------------------------------------------------
// Kernels. V == 0 selects the two-pass generic path.

template <int V, bool VEC>
__global__ __launch_bounds__(kMaxRowThreads) void rmsnorm_kernel(float *out, const float *in,
                                                                 const float *weight, int size,
                                                                 float eps) {
  __shared__ float slots[32];
  const size_t off = static_cast<size_t>(blockIdx.x) * size;
  if constexpr (V == 0)
    rmsnorm_row_generic(out + off, in + off, weight, size, eps, slots);
  else
    rmsnorm_row<V, VEC>(out + off, in + off, weight, size, eps, slots);
}

template <int V, bool VEC>
__global__ __launch_bounds__(kMaxRowThreads) void softmax_kernel(float *out, const float *logits,
                                                                 int size) {
  __shared__ float slots[32];
  const size_t off = static_cast<size_t>(blockIdx.x) * size;
  if constexpr (V == 0)
    softmax_row_generic(out + off, logits + off, size, slots);
  else
    softmax_row<V, VEC>(out + off, logits + off, size, slots);
}

// One launch for a whole llama2c iteration. Block b handles:
//   b < 2*pairs           rmsnorm row b/2 (even b) or softmax row b/2 (odd b)
//   then                  the remaining rmsnorm rows, then remaining softmax rows
//   then                  matrix-vector rows
// so the short matrix-vector blocks fill the tail of the launch.
template <int V, bool VEC>
__global__ __launch_bounds__(kFusedThreads) void fused_kernel(
    float *normalized, const float *input, const float *weight, float *softmax,
    const float *logits, float *product, const float *matrix, int size, int rms_rows,
    int softmax_rows, float eps) {
  __shared__ float slots[32];
  int item = blockIdx.x;
  const int pairs = min(rms_rows, softmax_rows);
  int kind, row;
  if (item < 2 * pairs) {
    kind = item & 1;
    row = item >> 1;
  } else if ((item -= 2 * pairs) < rms_rows - pairs) {
    kind = 0;
    row = pairs + item;
  } else if ((item -= rms_rows - pairs) < softmax_rows - pairs) {
    kind = 1;
    row = pairs + item;
  } else {
    kind = 2;
    row = item - (softmax_rows - pairs);
  }
  const size_t off = static_cast<size_t>(row) * size;
  if constexpr (V == 0) {
    if (kind == 0) rmsnorm_row_generic(normalized + off, input + off, weight, size, eps, slots);
    else if (kind == 1) softmax_row_generic(softmax + off, logits + off, size, slots);
    else matvec_row_block_generic(product + row, matrix + off, input, size, slots);
  } else {
    if (kind == 0) rmsnorm_row<V, VEC>(normalized + off, input + off, weight, size, eps, slots);
    else if (kind == 1) softmax_row<V, VEC>(softmax + off, logits + off, size, slots);
    else matvec_row_block<V, VEC>(product + row, matrix + off, input, size, slots);
  }
}

// Reference structure: one lane per output row, columns in order, one fused
// multiply-add per column.
__global__ __launch_bounds__(256) void matvec_naive_kernel(float *out, const float *x,
                                                           const float *W, int cols, int rows) {
  const int row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  const float *w = W + static_cast<size_t>(row) * cols;
  float acc = 0.0f;
  for (int c = 0; c < cols; ++c) acc = fmaf(x[c], w[c], acc);
  out[row] = acc;
}

// One wavefront per output row; kWavesPerBlock rows per block.
constexpr int kMatvecWaves = 4;

template <bool VEC>
__global__ __launch_bounds__(kMatvecWaves * L2C_WAVE) void matvec_wave_kernel(
    float *out, const float *x, const float *W, int cols, int rows) {
  const int lane = threadIdx.x % L2C_WAVE;
  const int row = blockIdx.x * kMatvecWaves + threadIdx.x / L2C_WAVE;
  if (row >= rows) return;
  const float *w = W + static_cast<size_t>(row) * cols;
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  if constexpr (VEC) {
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const int cols4 = cols >> 2;
    int c = lane;
    // Four independent 1 KiB wave loads in flight per step.
    for (; c + 3 * L2C_WAVE < cols4; c += 4 * L2C_WAVE) {
      const float4 m0 = l2c::ld4_stream(w4 + c);
      const float4 m1 = l2c::ld4_stream(w4 + c + L2C_WAVE);
      const float4 m2 = l2c::ld4_stream(w4 + c + 2 * L2C_WAVE);
      const float4 m3 = l2c::ld4_stream(w4 + c + 3 * L2C_WAVE);
      const float4 v0 = x4[c], v1 = x4[c + L2C_WAVE];
      const float4 v2 = x4[c + 2 * L2C_WAVE], v3 = x4[c + 3 * L2C_WAVE];
      a0 = fmaf(m0.x, v0.x, a0); a0 = fmaf(m0.y, v0.y, a0);
      a0 = fmaf(m0.z, v0.z, a0); a0 = fmaf(m0.w, v0.w, a0);
      a1 = fmaf(m1.x, v1.x, a1); a1 = fmaf(m1.y, v1.y, a1);
      a1 = fmaf(m1.z, v1.z, a1); a1 = fmaf(m1.w, v1.w, a1);
      a2 = fmaf(m2.x, v2.x, a2); a2 = fmaf(m2.y, v2.y, a2);
      a2 = fmaf(m2.z, v2.z, a2); a2 = fmaf(m2.w, v2.w, a2);
      a3 = fmaf(m3.x, v3.x, a3); a3 = fmaf(m3.y, v3.y, a3);
      a3 = fmaf(m3.z, v3.z, a3); a3 = fmaf(m3.w, v3.w, a3);
    }
    for (; c < cols4; c += L2C_WAVE) {
      const float4 m0 = l2c::ld4_stream(w4 + c);
      const float4 v0 = x4[c];
      a0 = fmaf(m0.x, v0.x, a0); a0 = fmaf(m0.y, v0.y, a0);
      a0 = fmaf(m0.z, v0.z, a0); a0 = fmaf(m0.w, v0.w, a0);
    }
  } else {
    int c = lane;
    for (; c + 3 * L2C_WAVE < cols; c += 4 * L2C_WAVE) {
      a0 = fmaf(__builtin_nontemporal_load(w + c), x[c], a0);
      a1 = fmaf(__builtin_nontemporal_load(w + c + L2C_WAVE), x[c + L2C_WAVE], a1);
      a2 = fmaf(__builtin_nontemporal_load(w + c + 2 * L2C_WAVE), x[c + 2 * L2C_WAVE], a2);
      a3 = fmaf(__builtin_nontemporal_load(w + c + 3 * L2C_WAVE), x[c + 3 * L2C_WAVE], a3);
    }
    for (; c < cols; c += L2C_WAVE) a0 = fmaf(__builtin_nontemporal_load(w + c), x[c], a0);
  }
  const float acc = l2c::wave_sum((a0 + a1) + (a2 + a3));
  if (lane == 0) out[row] = acc;
}

// ---------------------------------------------------------------------------
// Launch configuration for the row kernels: the smallest V (float4 per lane)
// whose row fits in <= 256 lanes, else in <= 1024 lanes, else the generic
// two-pass path. Lanes are rounded up to whole wavefronts.

struct RowConfig {
  int threads;
  int v;  // 0 = generic
};

RowConfig choose_row_config(int size, int max_threads = kMaxRowThreads) {
  const int chunks = (size + 3) / 4;
  for (int limit : {256, max_threads}) {
    if (limit > max_threads) continue;
    for (int v = 1; v <= 16; v *= 2) {
      const int lanes = (chunks + v - 1) / v;
      const int threads = (lanes + L2C_WAVE - 1) / L2C_WAVE * L2C_WAVE;
      if (threads <= limit) return {threads, v};
    }
  }
  return {kGenericThreads, 0};
}

using RmsFn = void (*)(float *, const float *, const float *, int, float);
using SoftFn = void (*)(float *, const float *, int);
using FusedFn = void (*)(float *, const float *, const float *, float *, const float *, float *,
                         const float *, int, int, int, float);

int v_index(int v) {
  switch (v) {
    case 1: return 1;
    case 2: return 2;
    case 4: return 3;
    case 8: return 4;
    case 16: return 5;
    default: return 0;
  }
}

RmsFn rms_fn(int v, bool vec) {
  static const RmsFn fv[] = {rmsnorm_kernel<0, false>, rmsnorm_kernel<1, true>,
                             rmsnorm_kernel<2, true>,  rmsnorm_kernel<4, true>,
                             rmsnorm_kernel<8, true>,  rmsnorm_kernel<16, true>};
  static const RmsFn fs[] = {rmsnorm_kernel<0, false>, rmsnorm_kernel<1, false>,
                             rmsnorm_kernel<2, false>, rmsnorm_kernel<4, false>,
                             rmsnorm_kernel<8, false>, rmsnorm_kernel<16, false>};
  return vec ? fv[v_index(v)] : fs[v_index(v)];
}

SoftFn soft_fn(int v, bool vec) {
  static const SoftFn fv[] = {softmax_kernel<0, false>, softmax_kernel<1, true>,
                              softmax_kernel<2, true>,  softmax_kernel<4, true>,
                              softmax_kernel<8, true>,  softmax_kernel<16, true>};
  static const SoftFn fs[] = {softmax_kernel<0, false>, softmax_kernel<1, false>,
                              softmax_kernel<2, false>, softmax_kernel<4, false>,
                              softmax_kernel<8, false>, softmax_kernel<16, false>};
  return vec ? fv[v_index(v)] : fs[v_index(v)];
}

FusedFn fused_fn(int v, bool vec) {
  static const FusedFn fv[] = {fused_kernel<0, false>, fused_kernel<1, true>,
                               fused_kernel<2, true>,  fused_kernel<4, true>,
                               fused_kernel<8, true>,  fused_kernel<16, true>};
  static const FusedFn fs[] = {fused_kernel<0, false>, fused_kernel<1, false>,
                               fused_kernel<2, false>, fused_kernel<4, false>,
                               fused_kernel<8, false>, fused_kernel<16, false>};
  return vec ? fv[v_index(v)] : fs[v_index(v)];
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI

extern "C" int l2c_rmsnorm(float *out, const float *in, const float *weight, int size, int batch,
                           float eps, hipStream_t stream) {
  if (size <= 0 || batch < 0) return hipErrorInvalidValue;
  if (batch == 0) return hipSuccess;
  if (!out || !in || !weight) return hipErrorInvalidValue;
  const RowConfig cfg = choose_row_config(size);
  const bool vec = size % 4 == 0 && l2c_aligned16(out) && l2c_aligned16(in) &&
                   l2c_aligned16(weight);
  hipLaunchKernelGGL(rms_fn(cfg.v, vec), dim3(batch), dim3(cfg.threads), 0, stream, out, in,
                     weight, size, eps);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

extern "C" int l2c_softmax(float *out, const float *logits, int size, int batch,
                           hipStream_t stream) {
  if (size <= 0 || batch < 0) return hipErrorInvalidValue;
  if (batch == 0) return hipSuccess;
  if (!out || !logits) return hipErrorInvalidValue;
  const RowConfig cfg = choose_row_config(size);
  const bool vec = size % 4 == 0 && l2c_aligned16(out) && l2c_aligned16(logits);
  hipLaunchKernelGGL(soft_fn(cfg.v, vec), dim3(batch), dim3(cfg.threads), 0, stream, out, logits,
                     size);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

extern "C" int l2c_matvec(float *out, const float *x, const float *W, int cols, int rows,
                          int variant, hipStream_t stream) {
  if (cols <= 0 || rows < 0) return hipErrorInvalidValue;
  if (variant != L2C_MATVEC_NAIVE && variant != L2C_MATVEC_COALESCED) return hipErrorInvalidValue;
  if (rows == 0) return hipSuccess;
  if (!out || !x || !W) return hipErrorInvalidValue;
  if (variant == L2C_MATVEC_NAIVE) {
    hipLaunchKernelGGL(matvec_naive_kernel, dim3((rows + 63) / 64), dim3(64), 0, stream, out, x,
                       W, cols, rows);
  } else {
    const bool vec = cols % 4 == 0 && l2c_aligned16(x) && l2c_aligned16(W);
    const dim3 grid((rows + kMatvecWaves - 1) / kMatvecWaves), block(kMatvecWaves * L2C_WAVE);
    if (vec)
      hipLaunchKernelGGL(matvec_wave_kernel<true>, grid, block, 0, stream, out, x, W, cols, rows);
    else
      hipLaunchKernelGGL(matvec_wave_kernel<false>, grid, block, 0, stream, out, x, W, cols,
                         rows);
  }
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

extern "C" int l2c_fused(float *normalized, const float *input, const float *weight,
                         float *softmax, const float *logits, float *product,
                         const float *matrix, int size, int rms_rows, int softmax_rows,
                         int matmul_rows, float eps, hipStream_t stream) {
  if (size <= 0 || rms_rows < 0 || softmax_rows < 0 || matmul_rows < 0)
    return hipErrorInvalidValue;
  const long long items = static_cast<long long>(rms_rows) + softmax_rows + matmul_rows;
  if (items == 0) return hipSuccess;
  if (items > 0x7fffffffLL) return hipErrorInvalidValue;
  if (rms_rows > 0 && (!normalized || !input || !weight)) return hipErrorInvalidValue;
  if (softmax_rows > 0 && (!softmax || !logits)) return hipErrorInvalidValue;
  if (matmul_rows > 0 && (!product || !matrix || !input)) return hipErrorInvalidValue;
  const RowConfig cfg = choose_row_config(size, kFusedThreads);
  auto ok = [](const void *p) { return p == nullptr || l2c_aligned16(p); };
  const bool vec = size % 4 == 0 && ok(normalized) && ok(input) && ok(weight) && ok(softmax) &&
                   ok(logits) && ok(matrix);
  hipLaunchKernelGGL(fused_fn(cfg.v, vec), dim3(static_cast<unsigned>(items)), dim3(cfg.threads),
                     0, stream, normalized, input, weight, softmax, logits, product, matrix, size,
                     rms_rows, softmax_rows, eps);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

// Launch shapes of the other translation units' kernels.
int l2c_gemm_launch_shape(int batch, int cols, int rows, int *grid, int *block,
                          int *blocks_per_cu);
int l2c_qgemm_launch_shape(int fmt, int batch, int cols, int rows, int *grid, int *block,
                           int *blocks_per_cu);

extern "C" int l2c_launch_shape(int op, int batch, int cols, int rows, int variant, int *grid,
                                int *block, int *blocks_per_cu) {
  if (!grid || !block || !blocks_per_cu || cols <= 0 || batch < 0 || rows < 0)
    return hipErrorInvalidValue;
  const void *fn = nullptr;
  switch (op) {
    case L2C_OP_RMSNORM:
    case L2C_OP_SOFTMAX: {
      const RowConfig cfg = choose_row_config(cols);
      const bool vec = cols % 4 == 0;
      fn = op == L2C_OP_RMSNORM ? reinterpret_cast<const void *>(rms_fn(cfg.v, vec))
                                : reinterpret_cast<const void *>(soft_fn(cfg.v, vec));
      *grid = batch;
      *block = cfg.threads;
      break;
    }
    case L2C_OP_MATVEC:
      if (variant == L2C_MATVEC_NAIVE) {
        fn = reinterpret_cast<const void *>(matvec_naive_kernel);
        *grid = (rows + 63) / 64;
        *block = 64;
      } else if (variant == L2C_MATVEC_COALESCED) {
        fn = cols % 4 == 0 ? reinterpret_cast<const void *>(matvec_wave_kernel<true>)
                           : reinterpret_cast<const void *>(matvec_wave_kernel<false>);
        *grid = (rows + kMatvecWaves - 1) / kMatvecWaves;
        *block = kMatvecWaves * L2C_WAVE;
      } else {
        return hipErrorInvalidValue;
      }
      break;
    case L2C_OP_FUSED: {
      const RowConfig cfg = choose_row_config(cols, kFusedThreads);
      fn = reinterpret_cast<const void *>(fused_fn(cfg.v, cols % 4 == 0));
      *grid = 2 * batch + rows;
      *block = cfg.threads;
      break;
    }
    case L2C_OP_MATMUL:
      return l2c_gemm_launch_shape(batch, cols, rows, grid, block, blocks_per_cu);
    case L2C_OP_MATMUL_Q:
      return l2c_qgemm_launch_shape(variant, batch, cols, rows, grid, block, blocks_per_cu);
    default:
      return hipErrorInvalidValue;
  }
  return static_cast<int>(hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, fn, *block, 0));
}

extern "C" const char *l2c_strerror(int code) {
  if (code == 0) return "success";
  return hipGetErrorString(static_cast<hipError_t>(code));
}

extern "C" const char *l2c_version(void) { return "l2c 0.1 gfx950"; }
