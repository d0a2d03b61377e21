// The iteration runner: device buffers, three streams with fork/join events,
// hipGraph capture versus direct launches, and the timing protocol of
// llama2c/llama2c_cuda_graph.cu:260-517 (warm-up, auto launch count, event-
// timed back-to-back loop, 20 isolated single iterations), on HIP.
//
// Beyond the reference protocol, every operation is also timed alone on its
// own stream (K launches between two events) so the line carries each
// kernel's duration and its fraction of the MI355X bound (HBM bytes for
// rmsnorm, softmax and the matrix-vector product; fp32 or bf16 matrix-core
// FLOPs for the batched products).
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>

#include "../../include/l2c.h"
#include "l2c_host.h"

#if __has_include(<rocprofiler-sdk-roctx/roctx.h>)
#include <rocprofiler-sdk-roctx/roctx.h>
#define L2C_HAS_ROCTX 1
#else
#define L2C_HAS_ROCTX 0
#endif

namespace l2c_host {

namespace {

constexpr double kAutoTargetMs = 50.0;
constexpr int kAutoMinLaunches = 20;
constexpr int kAutoMaxLaunches = 5000;
constexpr int kSingleIterations = 20;
// Per-operation timing: at least this much back-to-back load before the
// windows (the matrix cores run about 6% slower for the first ~50 ms under
// load), then this many event windows of K launches, median taken.
constexpr double kOpWarmMs = 100.0;
constexpr int kOpWindows = 5;

// Ranges named like the reference's NVTX ranges (llama2c_cuda_graph.cu:164-176).
void range_push(const char *label) {
#if L2C_HAS_ROCTX
  roctxRangePushA(label);
#else
  (void)label;
#endif
}
void range_pop() {
#if L2C_HAS_ROCTX
  roctxRangePop();
#endif
}

struct Failure {
  std::string message;
};

#define HIP_OK(call)                                                                   \
  do {                                                                                 \
    const hipError_t e__ = (call);                                                     \
    if (e__ != hipSuccess) throw Failure{std::string(#call) + " failed: " + hipGetErrorString(e__)}; \
  } while (0)

#define L2C_OK(call)                                                                   \
  do {                                                                                 \
    const int e__ = (call);                                                            \
    if (e__ != 0) throw Failure{std::string(#call) + " failed: " + l2c_strerror(e__)}; \
  } while (0)

template <typename T>
struct DeviceBuffer {
  T *ptr = nullptr;
  size_t count = 0;
  void alloc(size_t n) {
    count = n;
    if (n > 0) HIP_OK(hipMalloc(reinterpret_cast<void **>(&ptr), n * sizeof(T)));
  }
  ~DeviceBuffer() {
    if (ptr) (void)hipFree(ptr);
  }
};

template <typename T>
struct PinnedBuffer {
  T *ptr = nullptr;
  void alloc(size_t n) {
    if (n > 0) HIP_OK(hipHostMalloc(reinterpret_cast<void **>(&ptr), n * sizeof(T), hipHostMallocDefault));
  }
  ~PinnedBuffer() {
    if (ptr) (void)hipHostFree(ptr);
  }
};

struct Streams {
  hipStream_t rms = nullptr, soft = nullptr, mm = nullptr;
  hipEvent_t fork = nullptr, rms_done = nullptr, soft_done = nullptr;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  hipEvent_t marks[kOpWindows + 1] = {};
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  ~Streams() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    for (hipEvent_t e : {fork, rms_done, soft_done, t0, t1})
      if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : marks)
      if (e) (void)hipEventDestroy(e);
    for (hipStream_t s : {rms, soft, mm})
      if (s) (void)hipStreamDestroy(s);
  }
};

double ms_since(std::chrono::steady_clock::time_point start) {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start).count();
}

}  // namespace

bool run(const Options &o, const Inputs &in, RunResult *res, std::vector<float> *normalized,
         std::vector<float> *softmax, std::vector<float> *product, QuantOperands *quant) {
  try {
    HIP_OK(hipSetDevice(o.device));
    hipDeviceProp_t prop;
    HIP_OK(hipGetDeviceProperties(&prop, o.device));
    res->device_name = prop.name;
    res->arch = prop.gcnArchName;
    res->cu_count = prop.multiProcessorCount;

    const Matmul mm = o.matmul;
    const bool batched = matmul_is_batched(mm);
    const bool quantized = matmul_is_quantized(mm);
    const int B = o.batch, S = o.size, R = o.rows;
    const size_t vec_elems = static_cast<size_t>(B) * S;
    const size_t mat_elems = static_cast<size_t>(R) * S;
    const size_t prod_elems = batched ? static_cast<size_t>(B) * R : static_cast<size_t>(R);
    if (quantized && S % 32 != 0) throw Failure{"mxfp4/fp8 variants need size % 32 == 0"};
    const bool scaled = matmul_is_scaled(mm);
    if (scaled && S % 128 != 0) throw Failure{"mxfp4s/fp8s variants need size % 128 == 0"};

    DeviceBuffer<float> d_input, d_weight, d_prob, d_softmax, d_matrix, d_normalized, d_product;
    DeviceBuffer<uint16_t> d_xbf16;
    DeviceBuffer<uint8_t> d_codes, d_scales8, d_workspace;
    DeviceBuffer<float> d_scales32;
    d_input.alloc(vec_elems);
    d_prob.alloc(vec_elems);
    d_weight.alloc(S);
    d_matrix.alloc(mat_elems);
    d_normalized.alloc(vec_elems);
    d_softmax.alloc(vec_elems);
    d_product.alloc(prod_elems);
    HIP_OK(hipMemcpy(d_input.ptr, in.input.data(), vec_elems * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_prob.ptr, in.probabilities.data(), vec_elems * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_weight.ptr, in.weight.data(), static_cast<size_t>(S) * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_matrix.ptr, in.matrix.data(), mat_elems * 4, hipMemcpyHostToDevice));

    // Quantized variants: bf16 activations and quantized weights are prepared
    // once on the device (setup, untimed), then copied back for the oracle.
    const void *q_scales = nullptr;
    const int qfmt = matmul_is_mxfp4(mm) ? L2C_Q_MXFP4 : L2C_Q_FP8;
    if (quantized) {
      d_xbf16.alloc(vec_elems);
      // The block-scaled variants quantize the activations into this
      // workspace on every iteration (inside l2c_matmul_qs).
      if (scaled) d_workspace.alloc(l2c_mxfp8_workspace_bytes(B, S));
      L2C_OK(l2c_to_bf16(d_xbf16.ptr, d_input.ptr, vec_elems, nullptr));
      if (matmul_is_mxfp4(mm)) {
        d_codes.alloc(mat_elems / 2);
        d_scales8.alloc(mat_elems / 32);
        L2C_OK(l2c_quantize_mxfp4(d_codes.ptr, d_scales8.ptr, d_matrix.ptr, R, S, nullptr));
        q_scales = d_scales8.ptr;
      } else {
        d_codes.alloc(mat_elems);
        d_scales32.alloc(R);
        L2C_OK(l2c_quantize_fp8(d_codes.ptr, d_scales32.ptr, d_matrix.ptr, R, S, nullptr));
        q_scales = d_scales32.ptr;
      }
      HIP_OK(hipDeviceSynchronize());
      quant->x_bf16.resize(vec_elems);
      HIP_OK(hipMemcpy(quant->x_bf16.data(), d_xbf16.ptr, vec_elems * 2, hipMemcpyDeviceToHost));
      quant->codes.resize(d_codes.count);
      HIP_OK(hipMemcpy(quant->codes.data(), d_codes.ptr, d_codes.count, hipMemcpyDeviceToHost));
      if (matmul_is_mxfp4(mm)) {
        quant->scales_e8.resize(d_scales8.count);
        HIP_OK(hipMemcpy(quant->scales_e8.data(), d_scales8.ptr, d_scales8.count, hipMemcpyDeviceToHost));
      } else {
        quant->scales_f32.resize(R);
        HIP_OK(hipMemcpy(quant->scales_f32.data(), d_scales32.ptr, static_cast<size_t>(R) * 4,
                         hipMemcpyDeviceToHost));
      }
    }

    PinnedBuffer<float> h_normalized, h_softmax, h_product;
    h_normalized.alloc(vec_elems);
    h_softmax.alloc(vec_elems);
    h_product.alloc(prod_elems);

    Streams st;
    HIP_OK(hipStreamCreateWithFlags(&st.rms, hipStreamNonBlocking));
    HIP_OK(hipStreamCreateWithFlags(&st.soft, hipStreamNonBlocking));
    HIP_OK(hipStreamCreateWithFlags(&st.mm, hipStreamNonBlocking));
    HIP_OK(hipEventCreateWithFlags(&st.fork, hipEventDisableTiming));
    HIP_OK(hipEventCreateWithFlags(&st.rms_done, hipEventDisableTiming));
    HIP_OK(hipEventCreateWithFlags(&st.soft_done, hipEventDisableTiming));
    HIP_OK(hipEventCreate(&st.t0));
    HIP_OK(hipEventCreate(&st.t1));

    // Waves: grid / (resident workgroups per CU x CUs), as
    // llama2c_cuda_graph.cu:318-336 defines them.
    auto waves = [&](int op, int variant) {
      int grid = 0, block = 0, per_cu = 0;
      L2C_OK(l2c_launch_shape(op, B, S, R, variant, &grid, &block, &per_cu));
      return per_cu > 0 ? static_cast<double>(grid) / (static_cast<double>(per_cu) * res->cu_count) : 0.0;
    };
    if (mm == Matmul::kFused) {
      res->rms_waves = res->softmax_waves = res->matmul_waves = waves(L2C_OP_FUSED, 0);
    } else {
      res->rms_waves = waves(L2C_OP_RMSNORM, 0);
      res->softmax_waves = waves(L2C_OP_SOFTMAX, 0);
      if (mm == Matmul::kNaive || mm == Matmul::kCoalesced)
        res->matmul_waves = waves(L2C_OP_MATVEC, mm == Matmul::kNaive ? L2C_MATVEC_NAIVE : L2C_MATVEC_COALESCED);
      else if (mm == Matmul::kBatched)
        res->matmul_waves = waves(L2C_OP_MATMUL, 0);
      else
        res->matmul_waves = waves(scaled ? L2C_OP_MATMUL_QS : L2C_OP_MATMUL_Q, qfmt);
    }

    // Algorithmic bytes and flops per launch of each operation.
    const double vec_bytes = static_cast<double>(vec_elems) * 4.0;
    res->rms.bytes = 2.0 * vec_bytes + S * 4.0;
    res->softmax.bytes = 2.0 * vec_bytes;
    if (!batched) {
      res->matmul.bytes = static_cast<double>(mat_elems) * 4.0 + (static_cast<double>(S) + R) * 4.0;
      res->matmul.flops = 2.0 * R * S;
    } else {
      const double wbytes = mm == Matmul::kBatched ? mat_elems * 4.0
                            : matmul_is_mxfp4(mm) ? mat_elems / 2.0 + mat_elems / 32.0
                                                   : mat_elems * 1.0 + R * 4.0;
      const double xbytes = vec_elems * (quantized ? 2.0 : 4.0);
      res->matmul.bytes = xbytes + wbytes + static_cast<double>(B) * R * 4.0;
      res->matmul.flops = 2.0 * B * R * static_cast<double>(S);
    }
    res->min_bytes_per_iter = o.repeats * (res->rms.bytes + res->softmax.bytes + res->matmul.bytes);
    res->matmul_flops_per_iter = o.repeats * res->matmul.flops;

    auto launch_rms = [&](hipStream_t s) {
      L2C_OK(l2c_rmsnorm(d_normalized.ptr, d_input.ptr, d_weight.ptr, S, B, kRmsEpsilon, s));
    };
    auto launch_softmax = [&](hipStream_t s) {
      L2C_OK(l2c_softmax(d_softmax.ptr, d_prob.ptr, S, B, s));
    };
    auto launch_matmul = [&](hipStream_t s) {
      switch (mm) {
        case Matmul::kNaive:
          L2C_OK(l2c_matvec(d_product.ptr, d_input.ptr, d_matrix.ptr, S, R, L2C_MATVEC_NAIVE, s));
          break;
        case Matmul::kCoalesced:
          L2C_OK(l2c_matvec(d_product.ptr, d_input.ptr, d_matrix.ptr, S, R, L2C_MATVEC_COALESCED, s));
          break;
        case Matmul::kBatched:
          L2C_OK(l2c_matmul(d_product.ptr, d_input.ptr, d_matrix.ptr, B, S, R, s));
          break;
        case Matmul::kMxfp4:
        case Matmul::kFp8:
          L2C_OK(l2c_matmul_q(d_product.ptr, d_xbf16.ptr, d_codes.ptr, q_scales, qfmt, B, S, R, s));
          break;
        case Matmul::kMxfp4s:
        case Matmul::kFp8s:
          L2C_OK(l2c_matmul_qs(d_product.ptr, d_xbf16.ptr, d_codes.ptr, q_scales, qfmt, B, S, R,
                               d_workspace.ptr, d_workspace.count, s));
          break;
        case Matmul::kFused:
          break;
      }
    };
    auto fused = [&](int rms_rows, int soft_rows, int mm_rows, hipStream_t s) {
      L2C_OK(l2c_fused(d_normalized.ptr, d_input.ptr, d_weight.ptr, d_softmax.ptr, d_prob.ptr,
                       d_product.ptr, d_matrix.ptr, S, rms_rows, soft_rows, mm_rows, kRmsEpsilon, s));
    };
    // Copy-mode downloads: hipMemcpyAsync as the reference does, or (hostwrite)
    // a kernel storing into the pinned host buffers.
    auto d2h = [&](float *dst, const float *src, size_t n, hipStream_t s) {
      if (o.host_write) L2C_OK(l2c_copy_to_host(dst, src, n * 4, s));
      else HIP_OK(hipMemcpyAsync(dst, src, n * 4, hipMemcpyDeviceToHost, s));
    };
    // Kernels l2c_copy_to_host launches for one download: one over the 16-byte
    // chunks when both pointers are 16-byte aligned, and one over the bytes
    // left after them (the same rule the copy applies).
    auto host_copy_kernels = [](const void *dst, const void *src, size_t bytes) {
      const bool aligned = (reinterpret_cast<uintptr_t>(dst) % 16 == 0) && (reinterpret_cast<uintptr_t>(src) % 16 == 0);
      const size_t chunked = aligned ? bytes / 16 * 16 : 0;
      return (chunked > 0 ? 1 : 0) + (chunked < bytes ? 1 : 0);
    };
    // Kernels one iteration launches (the block-scaled products launch their
    // activation quantizer too; hostwrite adds the copy kernels of the three
    // downloads).
    const int kernels_per_rep = mm == Matmul::kFused ? 1 : 3 + (scaled ? 1 : 0);
    const int host_write_kernels =
        o.copy_outputs && o.host_write
            ? host_copy_kernels(h_normalized.ptr, d_normalized.ptr, vec_elems * 4) +
                  host_copy_kernels(h_softmax.ptr, d_softmax.ptr, vec_elems * 4) +
                  host_copy_kernels(h_product.ptr, d_product.ptr, prod_elems * 4)
            : 0;
    const int kernels_per_iter_planned =
        kernels_per_rep * o.repeats + host_write_kernels +
        (o.copy_outputs ? (mm == Matmul::kFused && !o.one_stream ? 1 : 0) : 0);

    // One iteration. Three-stream variants: fork from the product's stream,
    // `repeats` x {rmsnorm | softmax | matmul} on their streams, copies on
    // the last repeat in copy mode, join back (llama2c_cuda_graph.cu:347-381).
    // Fused: one launch per repeat; in copy mode the last repeat runs the
    // rmsnorm rows first so their copy overlaps the softmax and matmul rows
    // on the side stream (llama2c_sota.cu:474-496).
    // onestream: the same work on the rmsnorm stream alone, in the same order,
    // with no fork/join events (an iteration form beyond the reference's).
    int kernels_per_iter = 0;
    auto enqueue_iteration = [&]() {
      kernels_per_iter = kernels_per_iter_planned;
      if (o.one_stream) {
        for (int rep = 0; rep < o.repeats; ++rep) {
          if (mm == Matmul::kFused) {
            fused(B, B, R, st.rms);
          } else {
            launch_matmul(st.rms);
            launch_rms(st.rms);
            launch_softmax(st.rms);
          }
        }
        if (o.copy_outputs) {
          d2h(h_normalized.ptr, d_normalized.ptr, vec_elems, st.rms);
          d2h(h_softmax.ptr, d_softmax.ptr, vec_elems, st.rms);
          d2h(h_product.ptr, d_product.ptr, prod_elems, st.rms);
        }
        return;
      }
      if (mm == Matmul::kFused) {
        for (int rep = 0; rep < o.repeats; ++rep) {
          if (!(o.copy_outputs && rep + 1 == o.repeats)) {
            fused(B, B, R, st.rms);
            continue;
          }
          HIP_OK(hipEventRecord(st.fork, st.rms));
          HIP_OK(hipStreamWaitEvent(st.soft, st.fork, 0));
          fused(B, 0, 0, st.rms);
          d2h(h_normalized.ptr, d_normalized.ptr, vec_elems, st.rms);
          fused(0, B, R, st.soft);
          d2h(h_softmax.ptr, d_softmax.ptr, vec_elems, st.soft);
          d2h(h_product.ptr, d_product.ptr, prod_elems, st.soft);
          HIP_OK(hipEventRecord(st.soft_done, st.soft));
          HIP_OK(hipStreamWaitEvent(st.rms, st.soft_done, 0));
        }
        return;
      }
      // Fork from and join back to the product's stream: the path from one
      // product to the next (product, join, fork, product) then stays on one
      // stream, and only the short rmsnorm and softmax rows wait on the other
      // streams' events. Same dependencies as forking from the rmsnorm stream
      // (llama2c_cuda_graph.cu:347-381); at C4 it saves the direct iteration
      // the two cross-stream hops the product would otherwise wait for.
      HIP_OK(hipEventRecord(st.fork, st.mm));
      HIP_OK(hipStreamWaitEvent(st.rms, st.fork, 0));
      HIP_OK(hipStreamWaitEvent(st.soft, st.fork, 0));
      for (int rep = 0; rep < o.repeats; ++rep) {
        // The product first: its workgroups take their CUs at once, and the
        // rmsnorm and softmax rows fill the slots its workgroups leave free
        // (the three streams are independent, so the order changes no result).
        launch_matmul(st.mm);
        launch_rms(st.rms);
        launch_softmax(st.soft);
        if (rep + 1 == o.repeats && o.copy_outputs) {
          d2h(h_normalized.ptr, d_normalized.ptr, vec_elems, st.rms);
          d2h(h_softmax.ptr, d_softmax.ptr, vec_elems, st.soft);
          d2h(h_product.ptr, d_product.ptr, prod_elems, st.mm);
        }
      }
      HIP_OK(hipEventRecord(st.rms_done, st.rms));
      HIP_OK(hipEventRecord(st.soft_done, st.soft));
      HIP_OK(hipStreamWaitEvent(st.mm, st.rms_done, 0));
      HIP_OK(hipStreamWaitEvent(st.mm, st.soft_done, 0));
    };
    // The stream an iteration starts and ends on: the product's for the
    // three-stream form, the rmsnorm stream for the one-stream and fused forms.
    const hipStream_t home = o.one_stream || mm == Matmul::kFused ? st.rms : st.mm;

    if (o.graph) {
      auto t = std::chrono::steady_clock::now();
      range_push("llama2c.graph_capture");
      HIP_OK(hipStreamBeginCapture(home, hipStreamCaptureModeGlobal));
      enqueue_iteration();
      HIP_OK(hipStreamEndCapture(home, &st.graph));
      range_pop();
      res->graph_capture_ms = ms_since(t);
      t = std::chrono::steady_clock::now();
      HIP_OK(hipGraphInstantiate(&st.exec, st.graph, nullptr, nullptr, 0));
      res->graph_instantiate_ms = ms_since(t);
      t = std::chrono::steady_clock::now();
      HIP_OK(hipGraphUpload(st.exec, home));
      HIP_OK(hipStreamSynchronize(home));
      res->graph_upload_ms = ms_since(t);
    } else {
      kernels_per_iter = kernels_per_iter_planned;
    }
    res->kernels_per_iter = kernels_per_iter;

    auto run_iteration = [&]() {
      if (o.graph) HIP_OK(hipGraphLaunch(st.exec, home));
      else enqueue_iteration();
    };
    auto synchronize_all = [&]() {
      HIP_OK(hipStreamSynchronize(st.rms));
      HIP_OK(hipStreamSynchronize(st.soft));
      HIP_OK(hipStreamSynchronize(st.mm));
    };

    // Warm-up for at least warmup_ms, each iteration synchronized
    // (llama2c_cuda_graph.cu:409-431); warmup_iters=N adds a floor of N
    // iterations. Both floors hold: a handful of iterations is not long
    // enough for the clocks to settle under the matrix-core load (the first
    // ~30 ms of a C4 loop run up to 12% slow).
    const auto warm_start = std::chrono::steady_clock::now();
    int warm = 0;
    do {
      range_push("llama2c.warmup");
      run_iteration();
      range_pop();
      synchronize_all();
      ++warm;
    } while (warm < o.warmup_iters || ms_since(warm_start) < o.warmup_ms);
    res->warmup_iterations = warm;
    int launches = o.launches;
    if (o.auto_launches) {
      const double per_iter = ms_since(warm_start) / warm;
      launches = static_cast<int>(std::fmin(kAutoMaxLaunches, std::fmax(kAutoMinLaunches, kAutoTargetMs / per_iter)));
    }
    res->launches = launches;

    // Back-to-back loop (llama2c_cuda_graph.cu:433-456).
    HIP_OK(hipEventRecord(st.t0, home));
    const auto wall_start = std::chrono::steady_clock::now();
    for (int i = 0; i < launches; ++i) {
      range_push("llama2c.iteration");
      run_iteration();
      range_pop();
    }
    res->submit_us = 1000.0 * ms_since(wall_start);
    HIP_OK(hipEventRecord(st.t1, home));
    synchronize_all();
    res->wall_ms = ms_since(wall_start);
    float gpu_ms = 0.0f;
    HIP_OK(hipEventElapsedTime(&gpu_ms, st.t0, st.t1));
    res->gpu_ms = gpu_ms;

    // Single iterations from an idle device; median (:457-479).
    std::vector<double> singles;
    for (int i = 0; i < kSingleIterations; ++i) {
      synchronize_all();
      range_push("llama2c.single");
      HIP_OK(hipEventRecord(st.t0, home));
      run_iteration();
      HIP_OK(hipEventRecord(st.t1, home));
      range_pop();
      HIP_OK(hipEventSynchronize(st.t1));
      float ms = 0.0f;
      HIP_OK(hipEventElapsedTime(&ms, st.t0, st.t1));
      singles.push_back(1000.0 * ms);
    }
    synchronize_all();
    std::sort(singles.begin(), singles.end());
    res->single_us = (singles[(kSingleIterations - 1) / 2] + singles[kSingleIterations / 2]) / 2.0;

    // Outputs of the last iteration: already on the host in copy mode.
    if (!o.copy_outputs) {
      d2h(h_normalized.ptr, d_normalized.ptr, vec_elems, st.rms);
      d2h(h_softmax.ptr, d_softmax.ptr, vec_elems, st.soft);
      d2h(h_product.ptr, d_product.ptr, prod_elems, st.mm);
      synchronize_all();
    }
    // The MXFP8 activations the block-scaled product used (the workspace
    // layout of include/l2c.h: row-major codes, then [S/128][Bp][4] scales).
    if (scaled) {
      quant->x_codes.resize(vec_elems);
      HIP_OK(hipMemcpy(quant->x_codes.data(), d_workspace.ptr, vec_elems, hipMemcpyDeviceToHost));
      const size_t off = (vec_elems + 255) / 256 * 256, bp = (static_cast<size_t>(B) + 3) / 4 * 4;
      std::vector<uint8_t> tiles(static_cast<size_t>(S / 128) * bp * 4);
      HIP_OK(hipMemcpy(tiles.data(), d_workspace.ptr + off, tiles.size(), hipMemcpyDeviceToHost));
      quant->x_scales.resize(vec_elems / 32);
      for (size_t b = 0; b < static_cast<size_t>(B); ++b)
        for (size_t j = 0; j < static_cast<size_t>(S / 32); ++j)
          quant->x_scales[b * (S / 32) + j] = tiles[((j / 4) * bp + b) * 4 + j % 4];
    }
    normalized->assign(h_normalized.ptr, h_normalized.ptr + vec_elems);
    softmax->assign(h_softmax.ptr, h_softmax.ptr + vec_elems);
    product->assign(h_product.ptr, h_product.ptr + prod_elems);

    // Per-operation timing: one operation alone on its own stream. It first
    // runs back to back for at least kOpWarmMs (synchronized every 32
    // launches so the queue stays short), then kOpWindows windows of k
    // launches follow back to back, each between two events; the median
    // window over k is the launch duration.
    const int k = std::max(5, std::min(launches, 200));
    for (hipEvent_t &e : st.marks)
      if (!e) HIP_OK(hipEventCreate(&e));
    auto time_op = [&](hipStream_t s, auto &&op) {
      const auto warm_start = std::chrono::steady_clock::now();
      do {
        for (int i = 0; i < 32; ++i) op(s);
        HIP_OK(hipStreamSynchronize(s));
      } while (ms_since(warm_start) < kOpWarmMs);
      HIP_OK(hipEventRecord(st.marks[0], s));
      for (int w = 0; w < kOpWindows; ++w) {
        for (int i = 0; i < k; ++i) op(s);
        HIP_OK(hipEventRecord(st.marks[w + 1], s));
      }
      HIP_OK(hipEventSynchronize(st.marks[kOpWindows]));
      double window_us[kOpWindows];
      for (int w = 0; w < kOpWindows; ++w) {
        float ms = 0.0f;
        HIP_OK(hipEventElapsedTime(&ms, st.marks[w], st.marks[w + 1]));
        window_us[w] = 1000.0 * ms / k;
      }
      std::sort(window_us, window_us + kOpWindows);
      return window_us[kOpWindows / 2];
    };
    range_push("llama2c.kernels");
    if (mm == Matmul::kFused) {
      res->rms.us = time_op(st.rms, [&](hipStream_t s) { fused(B, 0, 0, s); });
      res->softmax.us = time_op(st.soft, [&](hipStream_t s) { fused(0, B, 0, s); });
      res->matmul.us = time_op(st.mm, [&](hipStream_t s) { fused(0, 0, R, s); });
    } else {
      res->rms.us = time_op(st.rms, launch_rms);
      res->softmax.us = time_op(st.soft, launch_softmax);
      res->matmul.us = time_op(st.mm, launch_matmul);
    }
    range_pop();
    synchronize_all();
    return true;
  } catch (const Failure &f) {
    res->error = f.message;
    return false;
  }
}

std::string result_line(const Options &o, const RunResult &r, const Validation &v) {
  constexpr double kHbmPeakGbps = 8000.0;         // MI355X HBM3E
  constexpr double kFp32MfmaPeakTflops = 157.3;   // dense fp32 matrix
  constexpr double kBf16MfmaPeakTflops = 2500.0;  // dense bf16 matrix
  constexpr double kFp8MfmaPeakTflops = 5000.0;   // dense fp8 matrix (the block-scaled products)
  const double gpu_ms_per_iter = r.gpu_ms / r.launches;
  const double achieved_gbps = r.min_bytes_per_iter / (gpu_ms_per_iter * 1.0e6);
  auto gbps = [](const KernelTiming &t) { return t.us > 0 ? t.bytes / (t.us * 1.0e3) : 0.0; };
  const bool batched = matmul_is_batched(o.matmul);
  const double mm_tflops = r.matmul.us > 0 ? r.matmul.flops / (r.matmul.us * 1.0e6) : 0.0;
  const double mm_peak = o.matmul == Matmul::kBatched   ? kFp32MfmaPeakTflops
                         : matmul_is_scaled(o.matmul) ? kFp8MfmaPeakTflops
                                                      : kBf16MfmaPeakTflops;
  const double mm_frac = batched ? mm_tflops / mm_peak : gbps(r.matmul) / kHbmPeakGbps;
  const double strict_product = matmul_is_quantized(o.matmul) ? 2.0e-3 : 1.0e-4 * std::sqrt(static_cast<double>(o.size));
  const bool strict_valid = v.valid && v.rms_max_rel_error <= 1.0e-5 && v.softmax_max_rel_error <= 1.0e-5 &&
                            v.product_max_rel_error <= strict_product;
  const double min_waves = std::fmin(r.rms_waves, std::fmin(r.softmax_waves, r.matmul_waves));
  char buf[4096];
  std::snprintf(
      buf, sizeof(buf),
      "mode=%s matmul=%s launches=%d batch=%d size=%d rows=%d repeats=%d copies=%d warmup_ms=%d "
      "warmup_iterations=%d gpu_ms=%.6f gpu_ms_per_iter=%.6f single_iterations=%d single_us=%.3f "
      "wall_ms=%.6f wall_ms_per_iter=%.6f submit_us=%.3f submit_us_per_iter=%.3f "
      "graph_capture_ms=%.6f graph_instantiate_ms=%.6f graph_upload_ms=%.6f rms_waves=%.3f "
      "softmax_waves=%.3f matmul_waves=%.3f min_waves=%.3f min_bytes_per_iter=%.0f "
      "achieved_gbps=%.1f valid=%d inputs=%s seed=%llu kernels_per_iter=%d "
      "device=%s arch=%s cus=%d rms_us=%.3f rms_gbps=%.1f rms_hbm_frac=%.4f softmax_us=%.3f "
      "softmax_gbps=%.1f softmax_hbm_frac=%.4f matmul_us=%.3f matmul_gbps=%.1f matmul_tflops=%.3f "
      "matmul_bound=%s matmul_frac=%.4f rms_max_rel_err=%.3e softmax_max_rel_err=%.3e "
      "product_max_rel_err=%.3e product_max_tol_ratio=%.3e check_vectors=%zu strict_valid=%d "
      "matmul_within_iter=%d product_bf16_act_rel_err=%.3e one_stream=%d host_write=%d",
      o.graph ? "graph" : "direct", matmul_name(o.matmul), r.launches, o.batch, o.size, o.rows,
      o.repeats, o.copy_outputs ? 1 : 0, o.warmup_ms, r.warmup_iterations, r.gpu_ms, gpu_ms_per_iter,
      kSingleIterations, r.single_us, r.wall_ms, r.wall_ms / r.launches, r.submit_us,
      r.submit_us / r.launches, r.graph_capture_ms, r.graph_instantiate_ms, r.graph_upload_ms,
      r.rms_waves, r.softmax_waves, r.matmul_waves, min_waves, r.min_bytes_per_iter, achieved_gbps,
      v.valid ? 1 : 0, input_name(o.inputs.mode),
      static_cast<unsigned long long>(o.inputs.mode == InputMode::kDeterministic ? 0 : o.inputs.seed),
      r.kernels_per_iter, r.device_name.empty() ? "?" : r.device_name.c_str(),
      r.arch.empty() ? "?" : r.arch.substr(0, r.arch.find(':')).c_str(), r.cu_count, r.rms.us,
      gbps(r.rms), gbps(r.rms) / kHbmPeakGbps, r.softmax.us, gbps(r.softmax),
      gbps(r.softmax) / kHbmPeakGbps, r.matmul.us, gbps(r.matmul), mm_tflops,
      batched ? "mfma" : "hbm", mm_frac, v.rms_max_rel_error, v.softmax_max_rel_error,
      v.product_max_rel_error, v.product_max_ratio,
      batched ? v.product.sampled_batch_rows.size() : static_cast<size_t>(1), strict_valid ? 1 : 0,
      r.matmul.us <= gpu_ms_per_iter * 1000.0 ? 1 : 0, v.product_bf16_act_rel_error, o.one_stream ? 1 : 0,
      o.host_write ? 1 : 0);
  std::string line = buf;
  // Device names may contain spaces; keep the line space-separated key=value.
  const size_t d = line.find(" device=");
  if (d != std::string::npos) {
    const size_t end = line.find(" arch=", d);
    for (size_t i = d + 8; i < end; ++i)
      if (line[i] == ' ') line[i] = '_';
  }
  return line;
}

}  // namespace l2c_host
