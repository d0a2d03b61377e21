// l2c_kernel_bench: launches one operation of the C ABI alone, N times, on
// device-resident inputs, and prints its average duration (HIP events) and
// achieved rate. It is the isolate mode of a profiling run: run it under
// `rocprofv3 --kernel-trace --stats` or `--pmc FETCH_SIZE` to attribute
// time and HBM bytes to a single kernel (llama2c/profile_cuda.sh:136-167
// isolates kernels the same way with ncu).
//
//   l2c_kernel_bench OP BATCH SIZE ROWS ITERS   (after >= 100 ms of warm-up launches)
//   OP: rmsnorm softmax gemv naive fused matmul mxfp4 fp8 copy vendor_f32 vendor_bf16
//       mxfp4s fp8s (the block-scaled product: MXFP8 activation quantizer +
//       scaled contraction, as l2c_matmul_qs runs them; cvt_mxfp8 the
//       quantizer alone; mxfp4s_narrow the same MXFP4 product with the scale
//       array 4 bytes past a 16-byte boundary, which l2c_matmul_qs runs on its
//       256 x 128 tile instead of the 128 x 256 one)
//       bf16 mxfp6 (lowprec classifier contractions, alpha on for bf16)
//       cvt_bf16 cvt_mxfp6 cvt_nvfp4 (lowprec per-step activation conversions
//       of BATCH x SIZE; cvt_nvfp4 = tensor scales + codes + bf16 expansion)
//
// `copy` runs a plain 16-byte-per-lane copy of BATCH x SIZE floats (read
// once, written once): the calibration kernel for the FETCH_SIZE/WRITE_SIZE
// counters.
//
// `gemv_cold` times the coalesced matrix-vector product with the 256 MB
// Infinity Cache (MALL) flushed before every launch by a read-only sweep of
// 1 GiB (ordinary loads, nothing written), so no dirty line is left to be
// written back while the product is timed; only the product is bracketed by
// events, so its time is HBM's rate for W, not a MALL hit's (`gemv` runs back
// to back, where a W of up to ~256 MB stays in the MALL between launches).
// `gemv_cold_copy` flushes with a 1 GiB copy instead (512 MiB read, 512 MiB
// written), the form that leaves dirty lines behind. `read_cold` times the
// read-only sweep kernel itself over W's bytes after the same flush: a plain
// streaming read of that many bytes from HBM, the rate an isolated product of
// that size can hope for. `rmsnorm_cold` and `softmax_cold` time the row
// kernels after the same read-only flush, so their rows come from HBM; run
// back to back (`rmsnorm`, `softmax`), a 64 MiB input stays in the MALL.
// `copy_cold` is the plain copy of BATCH x SIZE floats after that flush.
// `read` is the flush's read-only sweep over BATCH x SIZE floats, back to
// back: with up to ~256 MB the data stays in the MALL, so it is the rate the
// MALL delivers to the CUs (the ceiling of the back-to-back C2 product).
//
// `vendor_f32` and `vendor_bf16` time the vendor library's GEMM of the same
// contraction (hipBLASLt, out[b][r] = sum_k X[b][k] W[r][k] with fp32 or bf16
// operands, fp32 output and accumulation): the fastest of the library's first
// eight heuristic choices, picked by a short timing run, then timed like the
// other ops. They are comparison points only; the product never calls the
// library. A line `vendor_check` gives the largest difference from this
// library's own contraction over every output, relative to the largest
// output magnitude (both apply the bf16 op's alpha of 0.5).
//
// `stage_wstep`, `stage_wpair`, `stage_split64`, `stage_split128` and
// `stage_fp8` are staging-only copies of the block-scaled contractions' operand DMA
// (BATCH x SIZE E4M3 X codes, ROWS x SIZE E2M1 W codes; no matrix-core work,
// no fragment reads, no scales): 512-lane workgroups on an XCD-ordered tile
// map, LDS DMA of 16 bytes a lane issued three steps ahead of its wait, one
// barrier a step, as in the kernel. stage_wstep: 128 x 256 tiles, per
// 128-k step X 128 bytes and W 64 bytes a row; stage_wpair: the same with W
// 128 bytes a row every other step; stage_split64 and stage_split128: 256 x
// 256 tiles with k split over two workgroups, interleaved 64-k halves of every
// step (X 64 and W 32 bytes a row) or contiguous halves of k (X 128 and W 64
// bytes a row, three stages); stage_fp8: the fp8-weight kernel's 256 x 128
// tiles, per step X 128 bytes a row and 128 rows of E4M3 W 128 bytes a row,
// three stages. They time how the L2 serves each pattern of row segments;
// `bytes` is the bytes staged.
//
// `mfma_f8f4`, `mfma_f8f8` and `mfma_bf16` run the random-operand loop of
// `ceiling` below (E4M3 x E2M1, E4M3 x E4M3 scaled, bf16) as an op, with as
// many loop trips as the shape's 2 BATCH SIZE ROWS FLOPs need: the matrix
// cores' half of a contraction alone, beside the `stage_*` copies of its
// staging half (and, under `python -m l2c.power`, its power).
//
//   l2c_kernel_bench ceiling
// measures the matrix-core rate the contractions can reach: register-only
// loops (no memory traffic) of v_mfma_f32_32x32x2_f32, v_mfma_f32_16x16x4_f32, v_mfma_f32_32x32x16_bf16
// and the scaled v_mfma_scale_f32_32x32x64_f8f6f4 (E3M2 x E3M2, E4M3 x E2M1,
// E4M3 x E4M3), two waves per SIMD,
// eight independent accumulators, on constant and on random operands, and on
// random operands with one wave per SIMD (256-lane blocks). The
// random-operand rate is the one real data meets (the matrix cores' power
// draw depends on the operand bits).
//
//   l2c_kernel_bench lds
// measures the LDS read rate per CU that the contractions' fragment reads
// draw on: one 96 KB block per CU (so no two share a CU) reads a 64 KB LDS
// array with ds_read_b128 or ds_read_b64, eight loads in flight per wave
// between waits, at 4, 8 and 16 waves per CU; bytes per shader clock per CU
// from the shader cycle counter, the clock from the fixed-rate wall clock.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/l2c.h"
#include "../csrc/l2c_common.h"

#define CHECK(call)                                                                    \
  do {                                                                                 \
    const hipError_t e__ = (call);                                                     \
    if (e__ != hipSuccess) {                                                           \
      std::fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e__));         \
      std::exit(1);                                                                    \
    }                                                                                  \
  } while (0)
#define L2C(call)                                                                      \
  do {                                                                                 \
    const int e__ = (call);                                                            \
    if (e__ != 0) {                                                                    \
      std::fprintf(stderr, "%s failed: %s\n", #call, l2c_strerror(e__));              \
      std::exit(1);                                                                    \
    }                                                                                  \
  } while (0)

__global__ void copy_kernel(float4 *dst, const float4 *src, size_t n4) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride)
    dst[i] = src[i];
}

// Reads n4 float4s with ordinary (allocating) loads and writes nothing unless
// their sum is exactly `never` (the inputs are finite and the caller passes a
// value no sum reaches), so the loads cannot be dropped and no line is dirtied.
__global__ void sweep_kernel(const float4 *src, size_t n4, float never, float *sink) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  float acc = 0.0f;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const float4 v = src[i];
    acc += (v.x + v.y) + (v.z + v.w);
  }
  if (acc == never) sink[0] = acc;
}

// Fills n floats with a deterministic pattern in [-1, 1) scaled by `scale`.
// Staging-only copy of the block-scaled contraction's operand DMA: per step
// an X tile (XR rows x XB bytes, step stride XS) and every WEVERY steps a W
// tile (WR rows x WB bytes of K / WDIV-byte rows, stride WS) into LDS rings (STAGES X slots, WSLOTS
// W slots), issued STAGES - 1 steps ahead and waited for one step ahead. With
// SPLIT == 2 the workgroups 2 T, 2 T + 1 (after the XCD remap) take halves of
// tile T's k range: interleaved halves of every step or contiguous halves.
typedef __attribute__((address_space(3))) void stage_lds_ptr;
template <int XR, int XB, int XS, int WB, int WS, int WEVERY, int STAGES, int WSLOTS, int SPLIT, bool INTERLEAVE,
          int WR = 256, int WDIV = 2>
__device__ __forceinline__ void stage_body(const uint8_t *X, const uint8_t *W, int M, int N, int K, float *sink) {
  constexpr int kX = XR * XB, kW = WR * WB;
  constexpr int kXI = kX / 8192, kWI = kW / 8192;  // DMA instructions per wave
  constexpr int kOut = (STAGES - 2) * kXI + kWI * (WEVERY == 1 ? STAGES - 2 : 1);
  static_assert(kOut == 6 || kOut == 8, "wait counts");
  __shared__ __attribute__((aligned(1024))) unsigned char lds[STAGES * kX + WSLOTS * kW];
  const int wrowbytes = K / WDIV;  // E2M1 (2) or E4M3 (1) rows
  int v = blockIdx.x;
  const int total = gridDim.x;
  if (total % 8 == 0) v = (v % 8) * (total / 8) + v / 8;
  const int tile = v / SPLIT, kh = v % SPLIT;
  const int mtiles = M / XR;
  const int m0 = (tile % mtiles) * XR, n0 = (tile / mtiles) * WR;
  const int steps = K / 128 / (INTERLEAVE ? 1 : SPLIT);
  const int xk0 = INTERLEAVE ? kh * XB : kh * (K / SPLIT);
  const int wk0 = INTERLEAVE ? kh * WB : kh * (wrowbytes / SPLIT);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
  const __amdgpu_buffer_rsrc_t rx = l2c::buffer_rsrc(X + static_cast<size_t>(m0) * K, static_cast<uint32_t>(XR) * K);
  const __amdgpu_buffer_rsrc_t rw =
      l2c::buffer_rsrc(W + static_cast<size_t>(n0) * wrowbytes, static_cast<uint32_t>(WR) * wrowbytes);
  constexpr int xl = XB / 16, wl = WB / 16;  // lanes per row
  int xsrc[kXI], wsrc[kWI];
#pragma unroll
  for (int q = 0; q < kXI; ++q)
    xsrc[q] = ((64 / xl) * (kXI * wave + q) + lane / xl) * K + 16 * (lane % xl);
#pragma unroll
  for (int q = 0; q < kWI; ++q)
    wsrc[q] = ((64 / wl) * (kWI * wave + q) + lane / wl) * wrowbytes + 16 * (lane % wl);
  auto dma = [&](int t) {
    unsigned char *xb = lds + (t % STAGES) * kX;
#pragma unroll
    for (int q = 0; q < kXI; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (stage_lds_ptr *)(xb + (kXI * wave + q) * 1024), 16, xsrc[q],
                                               xk0 + XS * t, 0, 0);
    if (t % WEVERY == 0) {
      unsigned char *wb = lds + STAGES * kX + ((t / WEVERY) % WSLOTS) * kW;
#pragma unroll
      for (int q = 0; q < kWI; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (stage_lds_ptr *)(wb + (kWI * wave + q) * 1024), 16, wsrc[q],
                                                 wk0 + WS * (t / WEVERY), 0, 0);
    }
  };
  for (int t = 0; t < STAGES - 1; ++t) dma(min(t, steps - 1));
  for (int t = 0; t < steps; ++t) {
    dma(min(t + STAGES - 1, steps - 1));
    if constexpr (kOut == 6)
      asm volatile("s_waitcnt vmcnt(6)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
  }
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  if (threadIdx.x == 0 && lds[wave] == 123 && lds[77] == 45) *sink = 1.0f;  // keeps the LDS live
}
#define L2C_STAGE_KERNEL(name, ...)                                                                         \
  __global__ __launch_bounds__(512, 1) void name(const uint8_t *X, const uint8_t *W, int M, int N, int K, \
                                                 float *sink) {                                           \
    stage_body<__VA_ARGS__>(X, W, M, N, K, sink);                                                          \
  }
L2C_STAGE_KERNEL(stage_wstep_kernel, 128, 128, 128, 64, 64, 1, 4, 4, 1, false)
L2C_STAGE_KERNEL(stage_wpair_kernel, 128, 128, 128, 128, 128, 2, 4, 2, 1, false)
L2C_STAGE_KERNEL(stage_split64_kernel, 256, 64, 128, 32, 64, 1, 4, 4, 2, true)
L2C_STAGE_KERNEL(stage_split128_kernel, 256, 128, 128, 64, 64, 1, 3, 3, 2, false)
L2C_STAGE_KERNEL(stage_fp8_kernel, 256, 128, 128, 128, 128, 1, 3, 3, 1, false, 128, 1)

__global__ void fill_kernel(float *p, size_t n, unsigned seed, float scale) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    unsigned h = static_cast<unsigned>(i) * 2654435761u ^ seed;
    h ^= h >> 15;
    h *= 2246822519u;
    h ^= h >> 13;
    p[i] = (static_cast<float>(h >> 8) * (1.0f / 8388608.0f) - 1.0f) * scale;
  }
}

#define BLT(call)                                                                      \
  do {                                                                                 \
    const hipblasStatus_t e__ = (call);                                                \
    if (e__ != HIPBLAS_STATUS_SUCCESS) {                                               \
      std::fprintf(stderr, "%s failed: status %d\n", #call, static_cast<int>(e__));    \
      std::exit(1);                                                                    \
    }                                                                                  \
  } while (0)

// ---------------------------------------------------------------------------
// Vendor GEMM (comparison only). Column-major views of the row-major operands:
// W (R x K) is K x R and taken transposed, X (B x K) is K x B, out (B x R) is
// R x B.
struct VendorGemm {
  hipblasLtHandle_t handle = nullptr;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  void *workspace = nullptr;
  size_t workspace_bytes = 0;
  float alpha = 1.0f, beta = 0.0f;

  void run(float *out, const void *W, const void *X, hipStream_t s) const {
    BLT(hipblasLtMatmul(handle, desc, &alpha, W, la, X, lb, &beta, out, lc, out, lc, &algo, workspace,
                        workspace_bytes, s));
  }
};

static VendorGemm vendor_setup(bool bf16, int B, int K, int R, float *out, const void *W, const void *X,
                               hipStream_t s) {
  VendorGemm v;
  const hipDataType in = bf16 ? HIP_R_16BF : HIP_R_32F;
  BLT(hipblasLtCreate(&v.handle));
  BLT(hipblasLtMatmulDescCreate(&v.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  BLT(hipblasLtMatmulDescSetAttribute(v.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta));
  BLT(hipblasLtMatmulDescSetAttribute(v.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb));
  BLT(hipblasLtMatrixLayoutCreate(&v.la, in, K, R, K));
  BLT(hipblasLtMatrixLayoutCreate(&v.lb, in, K, B, K));
  BLT(hipblasLtMatrixLayoutCreate(&v.lc, HIP_R_32F, R, B, R));
  hipblasLtMatmulPreference_t pref = nullptr;
  BLT(hipblasLtMatmulPreferenceCreate(&pref));
  const uint64_t max_ws = uint64_t(256) << 20;
  BLT(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &max_ws,
                                            sizeof max_ws));
  hipblasLtMatmulHeuristicResult_t res[8];
  int n = 0;
  BLT(hipblasLtMatmulAlgoGetHeuristic(v.handle, v.desc, v.la, v.lb, v.lc, v.lc, pref, 8, res, &n));
  BLT(hipblasLtMatmulPreferenceDestroy(pref));
  if (n < 1) {
    std::fprintf(stderr, "hipBLASLt offers no algorithm for this GEMM\n");
    std::exit(1);
  }
  size_t most = 0;
  for (int i = 0; i < n; ++i) most = std::max(most, res[i].workspaceSize);
  if (most > 0) CHECK(hipMalloc(&v.workspace, most));
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  float best = 0.0f;
  int pick = -1;
  for (int i = 0; i < n; ++i) {
    if (res[i].state != HIPBLAS_STATUS_SUCCESS) continue;
    v.algo = res[i].algo;
    v.workspace_bytes = res[i].workspaceSize;
    for (int w = 0; w < 5; ++w) v.run(out, W, X, s);
    CHECK(hipEventRecord(a, s));
    for (int r = 0; r < 10; ++r) v.run(out, W, X, s);
    CHECK(hipEventRecord(b, s));
    CHECK(hipEventSynchronize(b));
    float ms = 0.0f;
    CHECK(hipEventElapsedTime(&ms, a, b));
    std::printf("vendor_candidate=%d us=%.3f workspace=%zu\n", i, 100.0 * ms, res[i].workspaceSize);
    if (pick < 0 || ms < best) best = ms, pick = i;
  }
  if (pick < 0) {
    std::fprintf(stderr, "hipBLASLt returned no usable algorithm\n");
    std::exit(1);
  }
  v.algo = res[pick].algo;
  v.workspace_bytes = res[pick].workspaceSize;
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  std::printf("vendor_pick=%d of %d\n", pick, n);
  return v;
}

// Largest |a - b| over n device outputs, relative to the largest |b|.
static double max_rel_diff(const float *a, const float *b, size_t n) {
  std::vector<float> ha(n), hb(n);
  CHECK(hipMemcpy(ha.data(), a, n * 4, hipMemcpyDeviceToHost));
  CHECK(hipMemcpy(hb.data(), b, n * 4, hipMemcpyDeviceToHost));
  double diff = 0.0, big = 0.0;
  for (size_t i = 0; i < n; ++i) {
    diff = std::max(diff, static_cast<double>(std::fabs(ha[i] - hb[i])));
    big = std::max(big, static_cast<double>(std::fabs(hb[i])));
  }
  return big > 0.0 ? diff / big : diff;
}

// ---------------------------------------------------------------------------
// Matrix-core ceilings.
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ unsigned mix32(unsigned x) {
  x ^= x >> 15;
  x *= 2246822519u;
  x ^= x >> 13;
  x *= 3266489917u;
  return x ^ (x >> 16);
}

enum {
  kCeilF32 = 0, kCeilBf16 = 1, kCeilFp6 = 2, kCeilF8F4 = 3, kCeilF8F8 = 4, kCeilF32x16 = 5,
  kCeilBf16x16 = 6, kCeilF8F4x16 = 7, kCeilF8F8x16 = 8  // the 16 x 16 shapes of the same types
};

// Each lane holds four operand sets; MFMA (q, t) multiplies set q by set
// (q + t) % 4 into accumulator t. RANDOM: operand bits from a hash (fp32 and
// bf16 values with exponents near 1, any 6-bit or 4-bit codes, E4M3 codes
// with the top exponent bit clear so that none is NaN); else a constant.
// The scaled types take the operand formats of the block-scaled C5 path:
// E4M3 x E2M1 (MXFP4 weights) and E4M3 x E4M3 (fp8 weights).
template <int TYPE, int RANDOM>
__global__ __launch_bounds__(512) void ceiling_kernel(float *out, int n) {
  const unsigned id = blockIdx.x * 512 + threadIdx.x;
  f32x16 c[8];
  for (int t = 0; t < 8; ++t)
    for (int v = 0; v < 16; ++v) c[t][v] = 0.0f;
  if constexpr (TYPE == kCeilF32x16) {
    float a[4], b[4];
    for (int q = 0; q < 4; ++q) {
      a[q] = RANDOM ? __uint_as_float((mix32(id * 8 + q) & 0x807fffffu) | 0x3f000000u) : 1.0f;
      b[q] = RANDOM ? __uint_as_float((mix32(id * 8 + q + 4) & 0x807fffffu) | 0x3f000000u) : 1.0f;
    }
    f32x4 d[8];
    for (int t = 0; t < 8; ++t) d[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < n; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int t = 0; t < 8; ++t) d[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q], b[(q + t) & 3], d[t], 0, 0, 0);
    for (int t = 0; t < 8; ++t) c[t][0] = d[t][0] + d[t][1] + d[t][2] + d[t][3];
  } else if constexpr (TYPE == kCeilF32) {
    float a[4], b[4];
    for (int q = 0; q < 4; ++q) {
      a[q] = RANDOM ? __uint_as_float((mix32(id * 8 + q) & 0x807fffffu) | 0x3f000000u) : 1.0f;
      b[q] = RANDOM ? __uint_as_float((mix32(id * 8 + q + 4) & 0x807fffffu) | 0x3f000000u) : 1.0f;
    }
    for (int i = 0; i < n; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int t = 0; t < 8; ++t) c[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[q], b[(q + t) & 3], c[t], 0, 0, 0);
  } else if constexpr (TYPE == kCeilBf16 || TYPE == kCeilBf16x16) {
    u32x4 a[4], b[4];
    for (int q = 0; q < 4; ++q)
      for (int v = 0; v < 4; ++v) {
        a[q][v] = RANDOM ? (mix32(id * 32 + q * 4 + v) & 0x83ff83ffu) | 0x3c003c00u : 0x3c003c00u;
        b[q][v] = RANDOM ? (mix32(id * 32 + 16 + q * 4 + v) & 0x83ff83ffu) | 0x3c003c00u : 0x3c003c00u;
      }
    for (int i = 0; i < n; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          if constexpr (TYPE == kCeilBf16) {
            c[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[q]),
                                                           __builtin_bit_cast(bf16x8, b[(q + t) & 3]), c[t], 0, 0, 0);
          } else {
            f32x4 d = {c[t][0], c[t][1], c[t][2], c[t][3]};
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[q]),
                                                        __builtin_bit_cast(bf16x8, b[(q + t) & 3]), d, 0, 0, 0);
            c[t][0] = d[0], c[t][1] = d[1], c[t][2] = d[2], c[t][3] = d[3];
          }
        }
  } else if constexpr (TYPE == kCeilFp6) {
    i32x8 a[4], b[4];
    for (int q = 0; q < 4; ++q)
      for (int v = 0; v < 8; ++v) {
        a[q][v] = v < 6 ? static_cast<int>(RANDOM ? mix32(id * 64 + q * 8 + v) : 0x30c30c30u) : 0;
        b[q][v] = v < 6 ? static_cast<int>(RANDOM ? mix32(id * 64 + 32 + q * 8 + v) : 0x30c30c30u) : 0;
      }
    for (int i = 0; i < n; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int t = 0; t < 8; ++t)
          c[t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[q], b[(q + t) & 3], c[t], 3, 3, 0, 127, 0, 127);
  } else {
    // A: 32 E4M3 codes a lane (1.0 = 0x38); B: 32 E2M1 codes in 4 VGPRs
    // (1.0 = 0x2) or 32 E4M3 codes.
    constexpr bool kFp4 = TYPE == kCeilF8F4 || TYPE == kCeilF8F4x16;
    constexpr bool k16 = TYPE == kCeilF8F4x16 || TYPE == kCeilF8F8x16;
    constexpr int kFmtB = kFp4 ? 4 : 0;
    i32x8 a[4], b[4];
    for (int q = 0; q < 4; ++q)
      for (int v = 0; v < 8; ++v) {
        a[q][v] = static_cast<int>(RANDOM ? mix32(id * 64 + q * 8 + v) & 0xbfbfbfbfu : 0x38383838u);
        const unsigned rb = mix32(id * 64 + 32 + q * 8 + v);
        b[q][v] = kFp4 ? (v < 4 ? static_cast<int>(RANDOM ? rb : 0x22222222u) : 0)
                       : static_cast<int>(RANDOM ? rb & 0xbfbfbfbfu : 0x38383838u);
      }
    for (int i = 0; i < n; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          if constexpr (!k16) {
            c[t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[q], b[(q + t) & 3], c[t], 0, kFmtB, 0, 127, 0, 127);
          } else {
            f32x4 d = {c[t][0], c[t][1], c[t][2], c[t][3]};
            d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[q], b[(q + t) & 3], d, 0, kFmtB, 0, 127, 0, 127);
            c[t][0] = d[0], c[t][1] = d[1], c[t][2] = d[2], c[t][3] = d[3];
          }
        }
  }
  float sum = 0.0f;
  for (int t = 0; t < 8; ++t)
    for (int v = 0; v < 16; ++v) sum += c[t][v];
  out[id] = sum;
}

// threads = 512: one block per CU is two waves per SIMD; 256: one wave per
// SIMD, the matrix core fed by a single wave.
template <int TYPE, int RANDOM>
static double ceiling_rate(float *out, int blocks, int n, int threads) {
  for (int w = 0; w < 3; ++w)
    hipLaunchKernelGGL((ceiling_kernel<TYPE, RANDOM>), dim3(blocks), dim3(threads), 0, nullptr, out, n);
  CHECK(hipGetLastError());
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  const int reps = 5;
  CHECK(hipEventRecord(a));
  for (int r = 0; r < reps; ++r)
    hipLaunchKernelGGL((ceiling_kernel<TYPE, RANDOM>), dim3(blocks), dim3(threads), 0, nullptr, out, n);
  CHECK(hipEventRecord(b));
  CHECK(hipEventSynchronize(b));
  float ms = 0.0f;
  CHECK(hipEventElapsedTime(&ms, a, b));
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  const double mnk = TYPE == kCeilF32                                 ? 32.0 * 32 * 2
                     : TYPE == kCeilF32x16                             ? 16.0 * 16 * 4
                     : TYPE == kCeilBf16                               ? 32.0 * 32 * 16
                     : TYPE == kCeilBf16x16                            ? 16.0 * 16 * 32
                     : TYPE == kCeilF8F4x16 || TYPE == kCeilF8F8x16 ? 16.0 * 16 * 128
                                                                       : 32.0 * 32 * 64;  // scaled: k = 64
  const double waves = threads / 64.0;
  const double flops = 2.0 * mnk * 32.0 * n * reps * blocks * waves;  // 32 MFMAs a loop trip
  return flops / (ms * 1e9);
}

template <int TYPE>
static void ceiling_line(const char *name, float *out, int blocks, int trips) {
  double rc = 0, rr = 0, r1 = 0;
  for (int rep = 0; rep < 2; ++rep) {  // the second pass is reported (clocks settled)
    rc = ceiling_rate<TYPE, 0>(out, blocks, trips, 512);
    rr = ceiling_rate<TYPE, 1>(out, blocks, trips, 512);
    r1 = ceiling_rate<TYPE, 1>(out, blocks, trips, 256);
  }
  std::printf("ceiling mfma=%s constant_tflops=%.1f random_tflops=%.1f random_one_wave_tflops=%.1f\n", name, rc, rr,
              r1);
}

// The random-operand loop of one MFMA type as an op: one 512-lane block per
// CU, `trips` loop trips; returns the loop's FLOPs.
static double launch_mfma_loop(const std::string &op, float *out, int blocks, int trips, hipStream_t s) {
  double mnk = 32.0 * 32 * 64;
  if (op == "mfma_f8f4") {
    hipLaunchKernelGGL((ceiling_kernel<kCeilF8F4, 1>), dim3(blocks), dim3(512), 0, s, out, trips);
  } else if (op == "mfma_f8f8") {
    hipLaunchKernelGGL((ceiling_kernel<kCeilF8F8, 1>), dim3(blocks), dim3(512), 0, s, out, trips);
  } else {
    hipLaunchKernelGGL((ceiling_kernel<kCeilBf16, 1>), dim3(blocks), dim3(512), 0, s, out, trips);
    mnk = 32.0 * 32 * 16;
  }
  return 2.0 * mnk * 32.0 * trips * blocks * 8.0;  // 32 MFMAs a trip, 8 waves a block
}

static int run_ceilings() {
  int cus = 0;
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  const int blocks = cus;  // one block per CU
  float *out = nullptr;
  CHECK(hipMalloc(&out, static_cast<size_t>(blocks) * 512 * 4));
  ceiling_line<kCeilF32>("fp32 32x32x2", out, blocks, 400);
  ceiling_line<kCeilBf16>("bf16 32x32x16", out, blocks, 2000);
  ceiling_line<kCeilFp6>("fp6 (E3M2, scaled) 32x32x64", out, blocks, 2000);
  ceiling_line<kCeilF8F4>("fp8 x fp4 (E4M3 x E2M1, scaled) 32x32x64", out, blocks, 1000);
  ceiling_line<kCeilF8F8>("fp8 x fp8 (E4M3 x E4M3, scaled) 32x32x64", out, blocks, 1000);
  ceiling_line<kCeilF32x16>("fp32 16x16x4", out, blocks, 800);
  ceiling_line<kCeilBf16x16>("bf16 16x16x32", out, blocks, 4000);
  ceiling_line<kCeilF8F4x16>("fp8 x fp4 (E4M3 x E2M1, scaled) 16x16x128", out, blocks, 2000);
  ceiling_line<kCeilF8F8x16>("fp8 x fp8 (E4M3 x E4M3, scaled) 16x16x128", out, blocks, 2000);
  CHECK(hipFree(out));
  return 0;
}

// LDS read rate. Every lane reads BYTES at offsets that are multiples of
// BYTES inside the 64 KB it initialises, so each access is in bounds; the
// reads are volatile so the loop cannot be folded.
template <int BYTES>
__global__ __launch_bounds__(1024) void lds_read_kernel(unsigned *out, unsigned long long *clk, int iters) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[96 * 1024];  // 64 KB used
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  const int t = threadIdx.x;
  for (int i = t * 4; i < 65536; i += blockDim.x * 4) *reinterpret_cast<unsigned *>(lds + i) = i * 2654435761u;
  __syncthreads();
  // ds_read takes an LDS byte address: the array's own address plus the offset.
  const unsigned base = static_cast<unsigned>(reinterpret_cast<uintptr_t>(lds));
  const unsigned long long c0 = clock64(), w0 = wall_clock64();
  unsigned acc = 0, off = (t * BYTES) & 65535u;
  for (int it = 0; it < iters; ++it) {
    if constexpr (BYTES == 16) {
      u32x4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        asm volatile("ds_read_b128 %0, %1" : "=v"(v[u]) : "v"(base + ((off + u * 4096u) & 65535u)) : "memory");
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int u = 0; u < 8; ++u) acc ^= v[u][0] ^ v[u][3];
    } else {
      u32x2 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        asm volatile("ds_read_b64 %0, %1" : "=v"(v[u]) : "v"(base + ((off + u * 4096u) & 65535u)) : "memory");
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int u = 0; u < 8; ++u) acc ^= v[u][0] ^ v[u][1];
    }
    off = (off + 32768u) & 65535u;
  }
  const unsigned long long c1 = clock64(), w1 = wall_clock64();
  out[blockIdx.x * blockDim.x + t] = acc;
  if (t == 0) {
    clk[2 * blockIdx.x] = c1 - c0;
    clk[2 * blockIdx.x + 1] = w1 - w0;
  }
}

static int run_lds() {
  int cus = 0, wall_khz = 0;
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  CHECK(hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, 0));
  const int iters = 4096;
  unsigned *out = nullptr;
  unsigned long long *clk = nullptr;
  CHECK(hipMalloc(&out, static_cast<size_t>(cus) * 1024 * 4));
  CHECK(hipMalloc(&clk, static_cast<size_t>(cus) * 2 * 8));
  std::vector<unsigned long long> h(2 * static_cast<size_t>(cus));
  for (int threads : {256, 512, 1024}) {
    for (int bytes : {16, 8}) {
      for (int pass = 0; pass < 2; ++pass) {  // the second pass is reported
        if (bytes == 16)
          hipLaunchKernelGGL(lds_read_kernel<16>, dim3(cus), dim3(threads), 0, nullptr, out, clk, iters);
        else
          hipLaunchKernelGGL(lds_read_kernel<8>, dim3(cus), dim3(threads), 0, nullptr, out, clk, iters);
        CHECK(hipGetLastError());
        CHECK(hipDeviceSynchronize());
      }
      CHECK(hipMemcpy(h.data(), clk, h.size() * 8, hipMemcpyDeviceToHost));
      std::vector<double> cycles, ghz;
      for (int b = 0; b < cus; ++b) {
        cycles.push_back(static_cast<double>(h[2 * b]));
        ghz.push_back(static_cast<double>(h[2 * b]) / (static_cast<double>(h[2 * b + 1]) / (wall_khz * 1e3)) / 1e9);
      }
      std::sort(cycles.begin(), cycles.end());
      std::sort(ghz.begin(), ghz.end());
      const double bytes_per_block = static_cast<double>(iters) * 8 * threads * bytes;
      std::printf("lds read=b%d waves_per_cu=%d bytes_per_clk_per_cu=%.1f clock_ghz=%.2f\n", bytes * 8, threads / 64,
                  bytes_per_block / cycles[cus / 2], ghz[cus / 2]);
    }
  }
  CHECK(hipFree(out));
  CHECK(hipFree(clk));
  return 0;
}

int main(int argc, char **argv) {
  if (argc == 2 && std::strcmp(argv[1], "ceiling") == 0) return run_ceilings();
  if (argc == 2 && std::strcmp(argv[1], "lds") == 0) return run_lds();
  if (argc != 6) {
    std::fprintf(stderr, "Usage: %s OP BATCH SIZE ROWS ITERS | %s ceiling | %s lds\n", argv[0], argv[0], argv[0]);
    return 2;
  }
  const std::string op = argv[1];
  const int B = std::atoi(argv[2]), S = std::atoi(argv[3]), R = std::atoi(argv[4]);
  const int iters = std::atoi(argv[5]);
  if (B <= 0 || S <= 0 || R <= 0 || iters <= 0) {
    std::fprintf(stderr, "bad shape\n");
    return 2;
  }
  const size_t vec = static_cast<size_t>(B) * S, mat = static_cast<size_t>(R) * S;
  float *x = nullptr, *p = nullptr, *w = nullptr, *m = nullptr, *o1 = nullptr, *o2 = nullptr, *prod = nullptr;
  const bool mfma_loop = op == "mfma_f8f4" || op == "mfma_f8f8" || op == "mfma_bf16";
  const bool needs_matrix = op != "rmsnorm" && op != "softmax" && op != "copy" && op != "rmsnorm_cold" &&
                            op != "softmax_cold" && op != "copy_cold" && op != "read" && !mfma_loop;
  const bool staging = op == "stage_wstep" || op == "stage_wpair" || op == "stage_split64" || op == "stage_split128" ||
                       op == "stage_fp8";
  if (staging && (B % 256 != 0 || R % 256 != 0 || S % 512 != 0 || static_cast<long long>(256) * S > 0x7fffffffLL)) {
    std::fprintf(stderr, "staging ops need BATCH %% 256 == 0, ROWS %% 256 == 0, SIZE %% 512 == 0\n");
    return 2;
  }
  CHECK(hipMalloc(&x, vec * 4));
  CHECK(hipMalloc(&p, vec * 4));
  CHECK(hipMalloc(&w, static_cast<size_t>(S) * 4));
  CHECK(hipMalloc(&o1, vec * 4));
  CHECK(hipMalloc(&o2, vec * 4));
  if (needs_matrix) {
    CHECK(hipMalloc(&m, mat * 4));
    CHECK(hipMalloc(&prod, static_cast<size_t>(B) * R * 4));
  }
  hipLaunchKernelGGL(fill_kernel, dim3(1024), dim3(256), 0, nullptr, x, vec, 1u, 1.0f);
  hipLaunchKernelGGL(fill_kernel, dim3(1024), dim3(256), 0, nullptr, p, vec, 2u, 1.0f);
  hipLaunchKernelGGL(fill_kernel, dim3(64), dim3(256), 0, nullptr, w, static_cast<size_t>(S), 3u, 0.5f);
  if (m) hipLaunchKernelGGL(fill_kernel, dim3(4096), dim3(256), 0, nullptr, m, mat, 4u, 1.0f / 128.0f);
  CHECK(hipGetLastError());

  uint16_t *xb = nullptr, *wb = nullptr;
  uint8_t *codes = nullptr, *sc8 = nullptr, *xq = nullptr, *xs = nullptr, *ws = nullptr;
  size_t ws_bytes = 0;
  float *sc32 = nullptr, *alpha = nullptr, *partials = nullptr, *tscales = nullptr;
  const bool vendor = op == "vendor_f32" || op == "vendor_bf16";
  if (op == "bf16" || op == "vendor_bf16" || op == "mxfp6" || op == "cvt_bf16" || op == "cvt_mxfp6" ||
      op == "cvt_nvfp4") {
    if (S % 128 != 0) {
      std::fprintf(stderr, "lowprec ops need SIZE %% 128 == 0\n");
      return 2;
    }
    CHECK(hipMalloc(&xb, vec * 2));
    CHECK(hipMalloc(&xq, vec));
    CHECK(hipMalloc(&xs, vec / 16));
    CHECK(hipMalloc(&alpha, 4));
    CHECK(hipMalloc(&tscales, 8));
    CHECK(hipMalloc(&partials, L2C_NVFP4_PARTIALS * 4));
    const float one = 0.5f;
    CHECK(hipMemcpy(alpha, &one, 4, hipMemcpyHostToDevice));
    if (op == "bf16" || op == "vendor_bf16") {
      CHECK(hipMalloc(&wb, mat * 2));
      L2C(l2c_to_bf16_x4(xb, x, static_cast<long long>(vec), nullptr));
      L2C(l2c_to_bf16_x4(wb, m, static_cast<long long>(mat), nullptr));
    } else if (op == "mxfp6") {
      size_t cb = 0, sb = 0;
      L2C(l2c_mxfp6_bytes(R, S, &cb, &sb));
      CHECK(hipMalloc(&codes, cb));
      CHECK(hipMalloc(&sc8, sb));
      L2C(l2c_quantize_mxfp6(xq, xs, x, B, S, nullptr));
      L2C(l2c_quantize_mxfp6(codes, sc8, m, R, S, nullptr));
    }
  }
  const bool narrow = op == "mxfp4s_narrow";
  const bool scaled = op == "mxfp4s" || op == "fp8s" || op == "cvt_mxfp8" || narrow;
  if (scaled) {
    ws_bytes = l2c_mxfp8_workspace_bytes(B, S);
    if (ws_bytes == 0) {
      std::fprintf(stderr, "block-scaled ops need SIZE %% 128 == 0\n");
      return 2;
    }
    CHECK(hipMalloc(&ws, ws_bytes));
  }
  if (op == "mxfp4" || op == "fp8" || scaled) {
    if (S % 32 != 0) {
      std::fprintf(stderr, "quantized ops need SIZE %% 32 == 0\n");
      return 2;
    }
    CHECK(hipMalloc(&xb, vec * 2));
    L2C(l2c_to_bf16(xb, x, vec, nullptr));
    if (op == "mxfp4" || op == "mxfp4s" || narrow) {
      CHECK(hipMalloc(&codes, mat / 2));
      // narrow: the scales start 4 bytes into their allocation (4-byte
      // aligned, as the C ABI requires, but not 16-byte aligned).
      CHECK(hipMalloc(&sc8, mat / 32 + (narrow ? 4 : 0)));
      if (narrow) sc8 += 4;
      L2C(l2c_quantize_mxfp4(codes, sc8, m, R, S, nullptr));
    } else {
      CHECK(hipMalloc(&codes, mat));
      CHECK(hipMalloc(&sc32, static_cast<size_t>(R) * 4));
      L2C(l2c_quantize_fp8(codes, sc32, m, R, S, nullptr));
    }
  }
  CHECK(hipDeviceSynchronize());

  hipStream_t s;
  CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  float *read_sink = nullptr;
  if (op == "read" || staging) CHECK(hipMalloc(&read_sink, 4));
  // mfma_*: the loop trips that do the shape's 2 BATCH SIZE ROWS FLOPs.
  int cus = 0, trips = 0;
  float *loop_out = nullptr;
  if (mfma_loop) {
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    CHECK(hipMalloc(&loop_out, static_cast<size_t>(cus) * 512 * 4));
    const double per_trip = 2.0 * (op == "mfma_bf16" ? 32.0 * 32 * 16 : 32.0 * 32 * 64) * 32.0 * cus * 8.0;
    trips = std::max(1, static_cast<int>(2.0 * B * static_cast<double>(mat) / per_trip + 0.5));
  }
  VendorGemm vg;
  if (vendor) {
    const bool bf = op == "vendor_bf16";
    vg = vendor_setup(bf, B, S, R, prod, bf ? static_cast<const void *>(wb) : m,
                      bf ? static_cast<const void *>(xb) : x, s);
    if (bf) vg.alpha = 0.5f;  // the bf16 op's alpha
  }
  double bytes = 0, flops = 0;
  auto launch = [&]() {
    if (op == "rmsnorm") {
      L2C(l2c_rmsnorm(o1, x, w, S, B, 1.0e-5f, s));
      bytes = 2.0 * vec * 4 + S * 4.0;
    } else if (op == "softmax") {
      L2C(l2c_softmax(o2, p, S, B, s));
      bytes = 2.0 * vec * 4;
    } else if (op == "gemv" || op == "naive") {
      L2C(l2c_matvec(prod, x, m, S, R, op == "gemv" ? L2C_MATVEC_COALESCED : L2C_MATVEC_NAIVE, s));
      bytes = mat * 4.0 + (S + static_cast<double>(R)) * 4;
      flops = 2.0 * mat;
    } else if (op == "fused") {
      L2C(l2c_fused(o1, x, w, o2, p, prod, m, S, B, B, R, 1.0e-5f, s));
      bytes = 4.0 * vec * 4 + S * 4.0 + mat * 4.0 + (S + static_cast<double>(R)) * 4;
    } else if (op == "matmul") {
      L2C(l2c_matmul(prod, x, m, B, S, R, s));
      bytes = (vec + mat + static_cast<double>(B) * R) * 4;
      flops = 2.0 * B * static_cast<double>(mat);
    } else if (op == "mxfp4" || op == "fp8") {
      L2C(l2c_matmul_q(prod, xb, codes, op == "mxfp4" ? static_cast<const void *>(sc8) : sc32,
                       op == "mxfp4" ? L2C_Q_MXFP4 : L2C_Q_FP8, B, S, R, s));
      bytes = vec * 2.0 + (op == "mxfp4" ? mat / 2.0 + mat / 32.0 : mat + R * 4.0) +
              static_cast<double>(B) * R * 4;
      flops = 2.0 * B * static_cast<double>(mat);
    } else if (op == "mxfp4s" || op == "fp8s" || narrow) {
      const bool mx = op != "fp8s";
      L2C(l2c_matmul_qs(prod, xb, codes, mx ? static_cast<const void *>(sc8) : sc32, mx ? L2C_Q_MXFP4 : L2C_Q_FP8, B,
                        S, R, ws, ws_bytes, s));
      bytes = vec * 2.0 + (mx ? mat / 2.0 + mat / 32.0 : mat + R * 4.0) + static_cast<double>(B) * R * 4;
      flops = 2.0 * B * static_cast<double>(mat);
    } else if (mfma_loop) {
      flops = launch_mfma_loop(op, loop_out, cus, trips, s);
      CHECK(hipGetLastError());
    } else if (op == "cvt_mxfp8") {
      L2C(l2c_quantize_mxfp8(ws, ws_bytes, xb, B, S, s));
      bytes = vec * (2.0 + 1.0 + 1.0 / 32);
    } else if (op == "bf16") {
      L2C(l2c_matmul_bf16(prod, xb, wb, alpha, B, S, R, s));
      bytes = (vec + static_cast<double>(mat)) * 2 + static_cast<double>(B) * R * 4;
      flops = 2.0 * B * static_cast<double>(mat);
    } else if (op == "mxfp6") {
      L2C(l2c_matmul_mxfp6(prod, xq, xs, codes, sc8, B, S, R, s));
      bytes = (vec + static_cast<double>(mat)) * (0.75 + 1.0 / 32) + static_cast<double>(B) * R * 4;
      flops = 2.0 * B * static_cast<double>(mat);
    } else if (op == "cvt_bf16") {
      L2C(l2c_to_bf16_x4(xb, x, static_cast<long long>(vec), s));
      bytes = vec * 6.0;
    } else if (op == "cvt_mxfp6") {
      L2C(l2c_quantize_mxfp6(xq, xs, x, B, S, s));
      bytes = vec * (4.0 + 0.75 + 1.0 / 32);
    } else if (op == "cvt_nvfp4") {
      L2C(l2c_nvfp4_tensor_scales(tscales, alpha, tscales + 1, x, static_cast<long long>(vec), partials, s));
      L2C(l2c_quantize_nvfp4(xq, xs, xb, x, tscales, B, S, s));
      bytes = vec * (4.0 + 4.0 + 0.5 + 1.0 / 16 + 2.0);
    } else if (op == "vendor_f32") {
      vg.run(prod, m, x, s);
      bytes = (vec + mat + static_cast<double>(B) * R) * 4;
      flops = 2.0 * B * static_cast<double>(mat);
    } else if (op == "vendor_bf16") {
      vg.run(prod, wb, xb, s);
      bytes = (vec + static_cast<double>(mat)) * 2 + static_cast<double>(B) * R * 4;
      flops = 2.0 * B * static_cast<double>(mat);
    } else if (staging) {
      // X: B x S bytes of x's allocation, W: R x S / 2 bytes of m's.
      const uint8_t *X8 = reinterpret_cast<const uint8_t *>(x), *W8 = reinterpret_cast<const uint8_t *>(m);
      const int tiles128 = (B / 128) * (R / 256), tiles256 = (B / 256) * (R / 256);
      if (op == "stage_wstep")
        hipLaunchKernelGGL(stage_wstep_kernel, dim3(tiles128), dim3(512), 0, s,
                           X8, W8, B, R, S, read_sink);
      else if (op == "stage_wpair")
        hipLaunchKernelGGL(stage_wpair_kernel, dim3(tiles128), dim3(512), 0,
                           s, X8, W8, B, R, S, read_sink);
      else if (op == "stage_fp8")
        hipLaunchKernelGGL(stage_fp8_kernel, dim3((B / 256) * (R / 128)), dim3(512), 0, s, X8, W8, B, R, S, read_sink);
      else if (op == "stage_split64")
        hipLaunchKernelGGL(stage_split64_kernel, dim3(2 * tiles256), dim3(512), 0,
                           s, X8, W8, B, R, S, read_sink);
      else
        hipLaunchKernelGGL(stage_split128_kernel, dim3(2 * tiles256), dim3(512),
                           0, s, X8, W8, B, R, S, read_sink);
      CHECK(hipGetLastError());
      // Every tile stages all of its X rows and W rows over the whole k range.
      bytes = op == "stage_wstep" || op == "stage_wpair" ? static_cast<double>(tiles128) * (128.0 * S + 256.0 * S / 2)
              : op == "stage_fp8" ? static_cast<double>((B / 256) * (R / 128)) * (256.0 * S + 128.0 * S)
                                  : static_cast<double>(tiles256) * (256.0 * S + 256.0 * S / 2);
    } else if (op == "read") {
      hipLaunchKernelGGL(sweep_kernel, dim3(4096), dim3(256), 0, s, reinterpret_cast<const float4 *>(x), vec / 4,
                         1.0e30f, read_sink);
      CHECK(hipGetLastError());
      bytes = vec * 4.0;
    } else if (op == "copy") {
      hipLaunchKernelGGL(copy_kernel, dim3(4096), dim3(256), 0, s, reinterpret_cast<float4 *>(o1),
                         reinterpret_cast<const float4 *>(x), vec / 4);
      CHECK(hipGetLastError());
      bytes = 2.0 * (vec / 4) * 16;
    } else {
      std::fprintf(stderr, "unknown op %s\n", op.c_str());
      std::exit(2);
    }
  };
  hipEvent_t t0, t1;
  CHECK(hipEventCreate(&t0));
  CHECK(hipEventCreate(&t1));
  if (op == "gemv_cold" || op == "gemv_cold_copy" || op == "read_cold" || op == "rmsnorm_cold" ||
      op == "softmax_cold" || op == "copy_cold") {
    constexpr size_t kFlush = size_t(1) << 30;  // 1 GiB: four times the MALL
    float4 *fa = nullptr, *fb = nullptr;
    float *sink = nullptr;
    CHECK(hipMalloc(&fa, kFlush));
    CHECK(hipMalloc(&sink, 4));
    CHECK(hipMemset(fa, 0, kFlush));
    const bool copy_flush = op == "gemv_cold_copy";
    if (copy_flush) CHECK(hipMalloc(&fb, kFlush / 2));
    // The flush: a read of 1 GiB, or a copy of 512 MiB into another 512 MiB.
    auto flush = [&]() {
      if (copy_flush)
        hipLaunchKernelGGL(copy_kernel, dim3(4096), dim3(256), 0, s, fb, fa, kFlush / 2 / 16);
      else
        hipLaunchKernelGGL(sweep_kernel, dim3(4096), dim3(256), 0, s, fa, kFlush / 16, -1.0f, sink);
      CHECK(hipGetLastError());
    };
    double total_ms = 0.0, flush_ms = 0.0;
    hipEvent_t f0;
    CHECK(hipEventCreate(&f0));
    for (int i = 0; i < iters + 3; ++i) {
      CHECK(hipEventRecord(f0, s));
      flush();
      CHECK(hipEventRecord(t0, s));
      if (op == "read_cold")
        hipLaunchKernelGGL(sweep_kernel, dim3(4096), dim3(256), 0, s, reinterpret_cast<const float4 *>(m), mat / 4,
                           1.0e30f, sink);
      else if (op == "rmsnorm_cold")
        L2C(l2c_rmsnorm(o1, x, w, S, B, 1.0e-5f, s));
      else if (op == "softmax_cold")
        L2C(l2c_softmax(o2, p, S, B, s));
      else if (op == "copy_cold")
        hipLaunchKernelGGL(copy_kernel, dim3(4096), dim3(256), 0, s, reinterpret_cast<float4 *>(o1),
                           reinterpret_cast<const float4 *>(x), vec / 4);
      else
        L2C(l2c_matvec(prod, x, m, S, R, L2C_MATVEC_COALESCED, s));
      CHECK(hipGetLastError());
      CHECK(hipEventRecord(t1, s));
      CHECK(hipEventSynchronize(t1));
      float ms = 0.0f, fms = 0.0f;
      CHECK(hipEventElapsedTime(&ms, t0, t1));
      CHECK(hipEventElapsedTime(&fms, f0, t0));
      if (i >= 3) total_ms += ms, flush_ms += fms;  // three untimed rounds first
    }
    const double us = 1000.0 * total_ms / iters;
    const double bytes = op == "read_cold"      ? mat * 4.0
                         : op == "rmsnorm_cold" ? 2.0 * vec * 4 + S * 4.0
                         : op == "softmax_cold" || op == "copy_cold" ? 2.0 * vec * 4
                                                : mat * 4.0 + (S + static_cast<double>(R)) * 4;
    std::printf("op=%s batch=%d size=%d rows=%d iters=%d avg_us=%.3f bytes=%.0f gbps=%.1f flush=%s flush_us=%.1f\n",
                op.c_str(), B, S, R, iters, us, bytes, bytes / (us * 1e3), copy_flush ? "copy_512MiB" : "read_1GiB",
                1000.0 * flush_ms / iters);
    CHECK(hipEventDestroy(f0));
    return 0;
  }
  // Warm-up of 100 ms (at least 3 and at most 1000 launches): the matrix cores reach their
  // steady clock only after some tens of milliseconds under load.
  int warm = 0;
  float warm_ms = 0.0f;
  CHECK(hipEventRecord(t0, s));
  while (warm < 3 || (warm_ms < 100.0f && warm < 1000)) {
    launch();
    ++warm;
    CHECK(hipEventRecord(t1, s));
    CHECK(hipEventSynchronize(t1));
    CHECK(hipEventElapsedTime(&warm_ms, t0, t1));
  }
  CHECK(hipEventRecord(t0, s));
  for (int i = 0; i < iters; ++i) launch();
  CHECK(hipEventRecord(t1, s));
  CHECK(hipEventSynchronize(t1));
  float ms = 0;
  CHECK(hipEventElapsedTime(&ms, t0, t1));
  const double us = 1000.0 * ms / iters;
  if (vendor) {
    // The same contraction by this library, for the vendor_check line.
    float *ref = nullptr;
    CHECK(hipMalloc(&ref, static_cast<size_t>(B) * R * 4));
    if (op == "vendor_f32") L2C(l2c_matmul(ref, x, m, B, S, R, s));
    else L2C(l2c_matmul_bf16(ref, xb, wb, alpha, B, S, R, s));
    CHECK(hipStreamSynchronize(s));
    std::printf("vendor_check max_rel_diff=%.3e\n", max_rel_diff(prod, ref, static_cast<size_t>(B) * R));
    CHECK(hipFree(ref));
  }
  std::printf("op=%s batch=%d size=%d rows=%d iters=%d warmup=%d avg_us=%.3f bytes=%.0f gbps=%.1f tflops=%.3f\n",
              op.c_str(), B, S, R, iters, warm, us, bytes, bytes / (us * 1e3), flops / (us * 1e6));
  return 0;
}
