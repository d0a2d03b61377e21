// Device-side helpers shared by the l2c kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <cfloat>
#include <cstdint>

#define L2C_WAVE 64

namespace l2c {

// Butterfly sum over the 64 lanes of a wavefront; every lane gets the total.
// __shfl_xor lowers to ds_swizzle / ds_bpermute, which use the LDS crossbar
// but no LDS allocation.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, L2C_WAVE);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, L2C_WAVE));
  return v;
}

// Block-wide reductions through one LDS slot per wave. Every thread returns
// the result. Each call site passes its own slot array, so two reductions in
// a row need no barrier between them. The cross-wave sum runs in wave order,
// so the result does not depend on scheduling.
__device__ __forceinline__ float block_sum(float v, float *slots) {
  v = wave_sum(v);
  const int waves = blockDim.x / L2C_WAVE;
  if (threadIdx.x % L2C_WAVE == 0) slots[threadIdx.x / L2C_WAVE] = v;
  __syncthreads();
  float total = 0.0f;
  for (int w = 0; w < waves; ++w) total += slots[w];
  return total;
}

__device__ __forceinline__ float block_max(float v, float *slots) {
  v = wave_max(v);
  const int waves = blockDim.x / L2C_WAVE;
  if (threadIdx.x % L2C_WAVE == 0) slots[threadIdx.x / L2C_WAVE] = v;
  __syncthreads();
  float m = -FLT_MAX;
  for (int w = 0; w < waves; ++w) m = fmaxf(m, slots[w]);
  return m;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16-byte loads and stores with the nontemporal hint: data touched once
// streams through the caches without displacing reused operands.
__device__ __forceinline__ float4 ld4_stream(const float4 *p) {
  const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st4_stream(float4 *p, float4 v) {
  const f32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<f32x4 *>(p));
}

// Raw buffer resource over [p, p + bytes). Loads through it take a 32-bit
// per-lane byte offset plus a wave-uniform byte offset held in a scalar
// register, so a loop that walks along K advances one SGPR per step and
// spends no vector instructions on addresses. Word 3 selects the 32-bit data
// format that untyped (raw) buffer loads require on gfx9-family parts.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

}  // namespace l2c

// Return code plumbing shared by the extern "C" entry points.
#define L2C_LAUNCH_CHECK()                      \
  do {                                          \
    hipError_t e__ = hipGetLastError();         \
    if (e__ != hipSuccess) return (int)e__;     \
  } while (0)

static inline bool l2c_aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// The quantized-weight kernel's bf16 form (l2c_qgemm.hip), for contractions
// whose K is not a multiple of 64.
int l2c_matmul_bf16_split(float *out, const uint16_t *X, const uint16_t *W, const float *alpha, int batch, int cols,
                          int rows, hipStream_t stream);
// The quantized-weight contraction for cols % 64 == 0 (l2c_qgemm_ks.hip),
// called by l2c_matmul_q after its argument checks.
int l2c_matmul_q_ks(float *out, const uint16_t *X, const uint8_t *Wq, const void *scales, int fmt, int batch,
                    int cols, int rows, hipStream_t stream);
// Workgroups of that kernel resident per CU (512-lane workgroups, one per
// tile: 256 x 128 for MXFP4, 128 x 256 for fp8).
int l2c_qgemm_ks_occupancy(int fmt, int *blocks_per_cu);
// Workgroups l2c_matmul_q_ks launches for this shape (its tile depends on fmt).
long long l2c_qgemm_ks_tiles(int fmt, int batch, int rows);
