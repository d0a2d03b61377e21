// Device-to-host copy by device stores: a kernel reads device memory and
// writes it straight into pinned host memory (hipHostMalloc; on ROCm its host
// address is also its device address) over the host link. The harness's
// `hostwrite` copy mode uses it in place of hipMemcpyAsync for the per-
// iteration output downloads of the reference's copy mode
// (llama2c/llama2c_cuda_graph.cu:369-374): inside a captured graph it is an
// ordinary kernel node rather than a memcpy node.
//
// 16-byte loads and stores, grid-stride; a tail of bytes % 16 (or any
// misaligned copy) goes byte by byte.
#include "l2c_common.h"
#include "../../include/l2c.h"

namespace {

constexpr int kThreads = 256;
constexpr int kBlocks = 1024;

__global__ __launch_bounds__(kThreads) void copy_to_host_kernel(uint4 *__restrict__ dst,
                                                                const uint4 *__restrict__ src, size_t n16) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

__global__ __launch_bounds__(kThreads) void copy_bytes_to_host_kernel(unsigned char *__restrict__ dst,
                                                                      const unsigned char *__restrict__ src,
                                                                      size_t n) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

}  // namespace

extern "C" int l2c_copy_to_host(void *host_dst, const void *src, size_t bytes, hipStream_t stream) {
  if (bytes == 0) return hipSuccess;
  if (!host_dst || !src) return hipErrorInvalidValue;
  const bool aligned = l2c_aligned16(host_dst) && l2c_aligned16(src);
  const size_t n16 = aligned ? bytes / 16 : 0;
  if (n16 > 0) {
    const size_t blocks = std::min<size_t>(kBlocks, (n16 + kThreads - 1) / kThreads);
    hipLaunchKernelGGL(copy_to_host_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, stream,
                       static_cast<uint4 *>(host_dst), static_cast<const uint4 *>(src), n16);
    L2C_LAUNCH_CHECK();
  }
  const size_t done = n16 * 16;
  if (done < bytes) {
    const size_t rest = bytes - done;
    const size_t blocks = std::min<size_t>(kBlocks, (rest + kThreads - 1) / kThreads);
    hipLaunchKernelGGL(copy_bytes_to_host_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, stream,
                       static_cast<unsigned char *>(host_dst) + done, static_cast<const unsigned char *>(src) + done,
                       rest);
    L2C_LAUNCH_CHECK();
  }
  return hipSuccess;
}
