// Batched fp32 contraction out[b][r] = sum_k W[r][k] * X[b][k] on the gfx950
// fp32 matrix cores (v_mfma_f32_32x32x2_f32).
//
// Shapes: X is M x K (M = batch), W is N x K (N = rows), out is M x N, all
// row-major, so both operands are K-contiguous. The contraction is the one of
// classifier_kernel, applications/loom_private/decoder/decoder.cu:79-125.
//
// Tiling (MI355X: 256 CUs, 8 XCDs with a 4 MiB L2 each, 160 KiB LDS per CU):
//  * A workgroup computes a BM x BN = 256 x 128 tile with 8 wavefronts of
//    64 x 64 each (2 x 2 MFMA blocks of 32 x 32). At the 1024 x 8192 x 16384
//    shape that is 4 x 64 = 256 tiles: one per CU, no tail.
//  * K advances in steps of BK = 32. Each step's A and B slabs are loaded from
//    global memory with 16-byte loads into registers while the previous slab
//    is multiplied out of LDS, then stored into the other half of a
//    double-buffered LDS ring: one barrier per step.
//  * LDS rows keep the operands' K-contiguous layout with a row stride of
//    BK + 4 floats, so the 16-byte fragment reads of 16 consecutive lanes hit
//    64 distinct banks.
//  * MFMA operand layout: for v_mfma_f32_32x32x2f32 lane l supplies
//    A[l % 32][k = l / 32] and B[k = l / 32][l % 32]. Because the contraction
//    sums over k, the k index may be permuted as long as A and B use the same
//    permutation: lane l reads four consecutive k values (one ds_read_b128)
//    from k0 + 4 * (l / 32), and MFMA t of four consumes the t-th of them.
//    Four MFMAs therefore cover 8 consecutive k with one LDS read per operand.
//  * Accumulator layout of the 32 x 32 block: register v of lane l holds
//    C[8 * (v / 4) + 4 * (l / 32) + v % 4][l % 32].
//  * XCD-aware order: workgroup i is dispatched to XCD i % 8. The tile order
//    is remapped so that each XCD owns a contiguous band of N tiles (all M
//    tiles of those rows of W): every W slab is fetched from HBM into one L2,
//    and X (64 MiB at the large shape) is shared by the 32 CUs of an XCD.
#include "l2c_common.h"
#include "../../include/l2c.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 256;
constexpr int kBN = 128;
constexpr int kBK = 32;
constexpr int kWavesM = 4;
constexpr int kWavesN = 2;
constexpr int kThreads = kWavesM * kWavesN * L2C_WAVE;  // 512
constexpr int kWaveM = kBM / kWavesM;                    // 64
constexpr int kWaveN = kBN / kWavesN;                    // 64
constexpr int kFragM = kWaveM / 32;                      // 2
constexpr int kFragN = kWaveN / 32;                      // 2
constexpr int kLdsStride = kBK + 4;                      // floats per LDS row
constexpr int kChunksPerRow = kBK / 4;                   // float4 per slab row
constexpr int kLoadsA = kBM * kChunksPerRow / kThreads;  // 4
constexpr int kLoadsB = kBN * kChunksPerRow / kThreads;  // 2
constexpr int kXcds = 8;

static_assert(kBM * kChunksPerRow % kThreads == 0, "A slab must split evenly");
static_assert(kBN * kChunksPerRow % kThreads == 0, "B slab must split evenly");
static_assert(kBK % 8 == 0, "BK must be a multiple of 8");

struct Smem {
  float a[2][kBM][kLdsStride];
  float b[2][kBN][kLdsStride];
};

// Loads one float4 of a K-contiguous operand row; zero outside
// [0, rows) x [0, K). Branch-free: the address is clamped into the operand
// and the value replaced afterwards, so every lane issues its load.
template <bool VEC>
__device__ __forceinline__ float4 load_chunk(const float *base, int row, int rows, int k, int K) {
  const bool row_ok = row < rows;
  const float *p = base + static_cast<size_t>(row_ok ? row : rows - 1) * K;
  if constexpr (VEC) {
    const bool ok = row_ok && k < K;
    const float4 v = *reinterpret_cast<const float4 *>(p + (k < K ? k : K - 4));
    return ok ? v : make_float4(0.f, 0.f, 0.f, 0.f);
  } else {
    float4 v;
    v.x = row_ok && k < K ? p[k] : 0.f;
    v.y = row_ok && k + 1 < K ? p[k + 1] : 0.f;
    v.z = row_ok && k + 2 < K ? p[k + 2] : 0.f;
    v.w = row_ok && k + 3 < K ? p[k + 3] : 0.f;
    return v;
  }
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void gemm_f32_mfma_kernel(float *__restrict__ out,
                                                                 const float *__restrict__ X,
                                                                 const float *__restrict__ W,
                                                                 int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) Smem sm;

  // XCD-aware tile order (see the file header).
  int tile = blockIdx.x;
  const int tiles = gridDim.x;
  if (tiles % kXcds == 0) tile = (tile % kXcds) * (tiles / kXcds) + tile / kXcds;
  const int mtiles = (M + kBM - 1) / kBM;
  const int m0 = (tile % mtiles) * kBM;
  const int n0 = (tile / mtiles) * kBN;

  const int t = threadIdx.x;
  const int lane = t % L2C_WAVE;
  const int wave = t / L2C_WAVE;
  const int wm = wave % kWavesM;
  const int wn = wave / kWavesM;

  float4 ga[kLoadsA], gb[kLoadsB];
  auto global_load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < kLoadsA; ++i) {
      const int idx = t + i * kThreads;
      ga[i] = load_chunk<VEC>(X, m0 + idx / kChunksPerRow, M, k0 + (idx % kChunksPerRow) * 4, K);
    }
#pragma unroll
    for (int i = 0; i < kLoadsB; ++i) {
      const int idx = t + i * kThreads;
      gb[i] = load_chunk<VEC>(W, n0 + idx / kChunksPerRow, N, k0 + (idx % kChunksPerRow) * 4, K);
    }
  };
  auto lds_store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kLoadsA; ++i) {
      const int idx = t + i * kThreads;
      *reinterpret_cast<float4 *>(&sm.a[buf][idx / kChunksPerRow][(idx % kChunksPerRow) * 4]) =
          ga[i];
    }
#pragma unroll
    for (int i = 0; i < kLoadsB; ++i) {
      const int idx = t + i * kThreads;
      *reinterpret_cast<float4 *>(&sm.b[buf][idx / kChunksPerRow][(idx % kChunksPerRow) * 4]) =
          gb[i];
    }
  };

  f32x16 acc[kFragM][kFragN];
#pragma unroll
  for (int i = 0; i < kFragM; ++i)
#pragma unroll
    for (int j = 0; j < kFragN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int frag_row = lane % 32;
  const int frag_k = 4 * (lane / 32);
  const int nk = (K + kBK - 1) / kBK;
  const float *a_base = &sm.a[0][wm * kWaveM + frag_row][frag_k];
  const float *b_base = &sm.b[0][wn * kWaveN + frag_row][frag_k];
  constexpr int kABuf = kBM * kLdsStride, kBBuf = kBN * kLdsStride;

  // Fragments of one 8-deep k group (one ds_read_b128 per operand block).
  float4 fa[2][kFragM], fb[2][kFragN];
  auto load_frags = [&](int slot, int buf, int kk) {
#pragma unroll
    for (int i = 0; i < kFragM; ++i)
      fa[slot][i] = *reinterpret_cast<const float4 *>(a_base + buf * kABuf + i * 32 * kLdsStride + kk);
#pragma unroll
    for (int j = 0; j < kFragN; ++j)
      fb[slot][j] = *reinterpret_cast<const float4 *>(b_base + buf * kBBuf + j * 32 * kLdsStride + kk);
  };
  auto mfma_group = [&](int slot) {
#pragma unroll
    for (int i = 0; i < kFragM; ++i)
#pragma unroll
      for (int j = 0; j < kFragN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[slot][i].x, fb[slot][j].x, acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < kFragM; ++i)
#pragma unroll
      for (int j = 0; j < kFragN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[slot][i].y, fb[slot][j].y, acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < kFragM; ++i)
#pragma unroll
      for (int j = 0; j < kFragN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[slot][i].z, fb[slot][j].z, acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < kFragM; ++i)
#pragma unroll
      for (int j = 0; j < kFragN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[slot][i].w, fb[slot][j].w, acc[i][j], 0, 0, 0);
  };

  global_load(0);
  lds_store(0);
  __syncthreads();
  load_frags(0, 0, 0);

  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) global_load((kt + 1) * kBK);
    // Fragments for group g + 1 are read while group g's MFMAs run.
#pragma unroll
    for (int g = 0; g < kBK / 8; ++g) {
      if (g + 1 < kBK / 8) load_frags((g + 1) & 1, buf, (g + 1) * 8);
      mfma_group(g & 1);
    }
    if (more) lds_store(buf ^ 1);
    __syncthreads();
    if (more) load_frags(0, buf ^ 1, 0);
  }

  // Epilogue: lanes 0-31 and 32-63 each write 32 consecutive floats of a row.
#pragma unroll
  for (int i = 0; i < kFragM; ++i) {
#pragma unroll
    for (int j = 0; j < kFragN; ++j) {
      const int n = n0 + wn * kWaveN + j * 32 + lane % 32;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * kWaveM + i * 32 + 8 * (v / 4) + 4 * (lane / 32) + v % 4;
        if (m < M && n < N) out[static_cast<size_t>(m) * N + n] = acc[i][j][v];
      }
    }
  }
}

}  // namespace

int l2c_gemm_launch_shape(int batch, int cols, int rows, int *grid, int *block,
                          int *blocks_per_cu) {
  *grid = ((batch + kBM - 1) / kBM) * ((rows + kBN - 1) / kBN);
  *block = kThreads;
  const void *fn = cols % 4 == 0 ? reinterpret_cast<const void *>(gemm_f32_mfma_kernel<true>)
                                 : reinterpret_cast<const void *>(gemm_f32_mfma_kernel<false>);
  return static_cast<int>(hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, fn, kThreads, 0));
}

extern "C" int l2c_matmul(float *out, const float *X, const float *W, int batch, int cols,
                          int rows, hipStream_t stream) {
  if (batch < 0 || cols <= 0 || rows < 0) return hipErrorInvalidValue;
  if (batch == 0 || rows == 0) return hipSuccess;
  if (!out || !X || !W) return hipErrorInvalidValue;
  const long long tiles =
      static_cast<long long>((batch + kBM - 1) / kBM) * ((rows + kBN - 1) / kBN);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  const bool vec = cols % 4 == 0 && l2c_aligned16(X) && l2c_aligned16(W);
  const dim3 grid(static_cast<unsigned>(tiles)), block(kThreads);
  if (vec)
    hipLaunchKernelGGL(gemm_f32_mfma_kernel<true>, grid, block, 0, stream, out, X, W, batch, rows,
                       cols);
  else
    hipLaunchKernelGGL(gemm_f32_mfma_kernel<false>, grid, block, 0, stream, out, X, W, batch,
                       rows, cols);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}
