// l2c_kernel_bench: launches one operation of the C ABI alone, N times, on
// device-resident inputs, and prints its average duration (HIP events) and
// achieved rate. It is the isolate mode of a profiling run: run it under
// `rocprofv3 --kernel-trace --stats` or `--pmc FETCH_SIZE` to attribute
// time and HBM bytes to a single kernel (llama2c/profile_cuda.sh:136-167
// isolates kernels the same way with ncu).
//
//   l2c_kernel_bench OP BATCH SIZE ROWS ITERS   (after >= 100 ms of warm-up launches)
//   OP: rmsnorm softmax gemv naive fused matmul mxfp4 fp8 copy
//       bf16 mxfp6 (lowprec classifier contractions, alpha on for bf16)
//       cvt_bf16 cvt_mxfp6 cvt_nvfp4 (lowprec per-step activation conversions
//       of BATCH x SIZE; cvt_nvfp4 = tensor scales + codes + bf16 expansion)
//
// `copy` runs a plain 16-byte-per-lane copy of BATCH x SIZE floats (read
// once, written once): the calibration kernel for the FETCH_SIZE/WRITE_SIZE
// counters.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/l2c.h"

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

// Fills n floats with a deterministic pattern in [-1, 1) scaled by `scale`.
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

int main(int argc, char **argv) {
  if (argc != 6) {
    std::fprintf(stderr, "Usage: %s OP BATCH SIZE ROWS ITERS\n", argv[0]);
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
  const bool needs_matrix = op != "rmsnorm" && op != "softmax" && op != "copy";
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
  uint8_t *codes = nullptr, *sc8 = nullptr, *xq = nullptr, *xs = nullptr;
  float *sc32 = nullptr, *alpha = nullptr, *partials = nullptr, *tscales = nullptr;
  if (op == "bf16" || op == "mxfp6" || op == "cvt_bf16" || op == "cvt_mxfp6" || op == "cvt_nvfp4") {
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
    if (op == "bf16") {
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
  if (op == "mxfp4" || op == "fp8") {
    if (S % 32 != 0) {
      std::fprintf(stderr, "quantized ops need SIZE %% 32 == 0\n");
      return 2;
    }
    CHECK(hipMalloc(&xb, vec * 2));
    L2C(l2c_to_bf16(xb, x, vec, nullptr));
    if (op == "mxfp4") {
      CHECK(hipMalloc(&codes, mat / 2));
      CHECK(hipMalloc(&sc8, mat / 32));
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
  std::printf("op=%s batch=%d size=%d rows=%d iters=%d warmup=%d avg_us=%.3f bytes=%.0f gbps=%.1f tflops=%.3f\n",
              op.c_str(), B, S, R, iters, warm, us, bytes, bytes / (us * 1e3), flops / (us * 1e6));
  return 0;
}
