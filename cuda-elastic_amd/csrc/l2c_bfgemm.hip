// bf16 x bf16 contraction with an optional device alpha:
//   out[b][r] = alpha * sum_k X[b][k] * W[r][k]
// (X batch x K, W rows x K, bf16 row-major; FP32 accumulation). The classifier
// of the lowprec bf16 case, and of the NVFP4 case on the exact bf16 expansions
// of its operands with alpha = d_X * d_W (experiments/blackwell/lowprec/
// spec.json "cases"; the reference runs CUTLASS GEMMs, decoder_lowprec.cu:82-121).
//
// Kernel design:
//  * v_mfma_f32_32x32x16_bf16. Tile 256 (batch) x 128 (rows) x 64 (k per step),
//    8 wavefronts: waves w and w + 4 share a SIMD and the same 128 x 64 output
//    sub-tile (4 x 2 blocks of 32 x 32); wave group g = w / 4 takes the step's
//    k-chunks q = 2g, 2g + 1 (lane (r, h) of MFMA q supplies k = 32h + 8q + 0..7
//    for both operands). Per step each wave reads 12 KB of fragments: 96 KB per
//    CU for 256 x 128 x 64 MACs at two waves per SIMD. The groups' partial sums
//    are added once at the end through LDS, group 1's before group 0's.
//  * LDS DMA staging (buffer_load ... lds, 16 B a lane, 1 KB = 8 rows a wave
//    instruction): 32 X and 16 W instructions a step, 6 per wave. LDS rows are
//    128 B with 16-byte chunks XOR-swizzled by row bits 1..3 (chunk c of row R
//    at slot c ^ ((R >> 1) & 7)); the DMA applies the swizzle on the source
//    side, so 16 lanes reading one chunk of 16 consecutive rows hit 16 distinct
//    slots of the 64 banks. Each of a lane's six instructions has its own
//    clamped per-lane source offset; the step's k offset is scalar.
//  * Ping-pong schedule (as in l2c_qgemm_ks.hip): the two waves of a SIMD run
//    half a step apart. A wave's memory phase of step t reads its fragments of
//    step t, issues the DMA of step t + 2 into the stage step t - 1 held and
//    waits for its DMA of step t + 1; its MFMA phase runs the step's 16 MFMAs at
//    raised wave priority. Group 0 (waves 0-3) and group 1 (waves 4-7) alternate
//    the phases with a workgroup barrier after each, so each SIMD's matrix core
//    takes one wave's MFMAs while the other wave reads LDS. Three stages (144
//    KB); a step's DMA has one step to land.
//  * Bounds, measured at 1024 x 16384 x 8192: the ping-pong form 227 against
//    239 µs for the earlier schedule (both waves of a SIMD in step, one
//    barrier a step; the matrix cores busy 58% of the time) on the same box;
//    waiting for the DMA a phase later, or no wave priority, measured the
//    same. Each memory phase moves about 72 KB through LDS (48 KB of fragment
//    reads, 24 KB of DMA), against 512 MFMA cycles.
//  * Every access is in bounds by construction (no reliance on buffer range
//    checks): lanes whose row is past the tile's rows load the last row instead
//    (those rows are never stored). K % 64 == 0; l2c_matmul_bf16 routes
//    K % 64 == 32 to the quantized-weight kernel's bf16 form.
#include "l2c_common.h"
#include "../../include/l2c.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_ptr;

constexpr int kBM = 256;
constexpr int kBN = 128;
constexpr int kThreads = 512;
constexpr int kStages = 3;
constexpr int kXBytes = kBM * 128;
constexpr int kWBytes = kBN * 128;
constexpr int kStage = kXBytes + kWBytes;  // 48 KB
constexpr int kLds = kStages * kStage;     // 144 KB; the partial-sum exchange needs 128 KB
constexpr int kXcds = 8;
static_assert(kBM * kBN * 4 <= kLds, "the exchange fits the stages");

__device__ __forceinline__ int swizzle(int row) { return (row >> 1) & 7; }

__global__ __launch_bounds__(kThreads, 1) void bf16_gemm_kernel(float *__restrict__ out,
                                                                const uint16_t *__restrict__ X,
                                                                const uint16_t *__restrict__ W,
                                                                const float *__restrict__ alpha, int M, int N,
                                                                int K) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[kLds];
  int tile = blockIdx.x;
  const int tiles = gridDim.x;
  if (tiles % kXcds == 0) tile = (tile % kXcds) * (tiles / kXcds) + tile / kXcds;
  const int mtiles = (M + kBM - 1) / kBM;
  const int m0 = (tile % mtiles) * kBM, n0 = (tile / mtiles) * kBN;
  const int mrows = min(kBM, M - m0), nrows = min(kBN, N - n0);
  const int tid = threadIdx.x, lane = tid % L2C_WAVE;
  const int wave = __builtin_amdgcn_readfirstlane(tid / L2C_WAVE);
  const int g = wave >> 2, p = wave & 3;
  const int wm = p & 1, wn = p >> 1;
  const int r = lane % 32, h = lane / 32;
  const int row_bytes = 2 * K;
  const __amdgpu_buffer_rsrc_t rx =
      l2c::buffer_rsrc(X + static_cast<size_t>(m0) * K, static_cast<uint32_t>(mrows) * row_bytes);
  const __amdgpu_buffer_rsrc_t rw =
      l2c::buffer_rsrc(W + static_cast<size_t>(n0) * K, static_cast<uint32_t>(nrows) * row_bytes);
  // DMA: instruction (block b of 8 rows) lane i fills row 8b + i / 8, slot i % 8
  // with chunk (i % 8) ^ swizzle(row). Block b = 8k + wave for X (k < 4) and
  // W (k < 2). The step's k offset is scalar; rows are clamped per lane.
  const int lrow = 8 * wave + lane / 8;  // the lane's row within the first block
  const int lchunk = 16 * ((lane % 8) ^ swizzle(lrow));
  int xsrc[4], wsrc[2];
#pragma unroll
  for (int k = 0; k < 4; ++k) xsrc[k] = min(64 * k + lrow, mrows - 1) * row_bytes + lchunk;
#pragma unroll
  for (int k = 0; k < 2; ++k) wsrc[k] = min(64 * k + lrow, nrows - 1) * row_bytes + lchunk;
  auto dma = [&](int stage, int t) __attribute__((always_inline)) {
    unsigned char *base = lds + stage * kStage;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr *)(base + (8 * k + wave) * 1024), 16, xsrc[k], 128 * t,
                                               0, 0);
#pragma unroll
    for (int k = 0; k < 2; ++k)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr *)(base + kXBytes + (8 * k + wave) * 1024), 16, wsrc[k],
                                               128 * t, 0, 0);
  };
  // This wave's DMA of the step before the newest has landed (six
  // instructions a step), its LDS reads are done; then the workgroup barrier.
  auto wait_dma_barrier = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  auto barrier = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  // Fragments: rows wm * 128 + 32 i + r (X) and wn * 64 + 32 j + r (W); chunk
  // 4h + q for q = 2g, 2g + 1. The swizzle of these rows is that of r.
  const int sw = swizzle(r);
  const int a0 = (wm * 128 + r) * 128, b0 = kXBytes + (wn * 64 + r) * 128;
  const int c0 = 16 * ((4 * h + 2 * g) ^ sw), c1 = 16 * ((4 * h + 2 * g + 1) ^ sw);
  u32x4 fa[4][2], fb[2][2];
  auto read = [&](int stage) __attribute__((always_inline)) {
    const unsigned char *base = lds + stage * kStage;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int c = q ? c1 : c0;
#pragma unroll
      for (int i = 0; i < 4; ++i) fa[i][q] = *reinterpret_cast<const u32x4 *>(base + a0 + 4096 * i + c);
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[j][q] = *reinterpret_cast<const u32x4 *>(base + b0 + 4096 * j + c);
    }
  };
  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int total = K / 64;
  const int last = total - 1;
  dma(0, 0);
  dma(1, min(1, last));
  wait_dma_barrier();  // step 0 landed everywhere
  if (g == 1) barrier();
  int cur = 0;
  for (int t = 0; t < total; ++t) {
    // Memory phase of step t: the fragment reads of step t, the DMA of step
    // t + 2 into the stage step t - 1 held, a wait for this wave's DMA of
    // step t + 1. Reads ahead of the DMA measured 1-2% faster than the DMA
    // first (221.6-224.3 against 225.4-226.4 µs at 1024 x 16384 x 8192).
    const int free_stage = cur == 0 ? kStages - 1 : cur - 1;
    read(cur);
    dma(free_stage, min(t + 2, last));
    wait_dma_barrier();
    // MFMA phase of step t.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fa[i][q]),
                                                              __builtin_bit_cast(bf16x8, fb[j][q]), acc[i][j], 0, 0,
                                                              0);
    __builtin_amdgcn_s_setprio(0);
    barrier();
    cur = cur == kStages - 1 ? 0 : cur + 1;
  }
  if (g == 0) barrier();

  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  float *exchange = reinterpret_cast<float *>(lds);
  if (g == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) exchange[((p * 8 + i * 2 + j) * 16 + v) * L2C_WAVE + lane] = acc[i][j][v];
  }
  __syncthreads();
  if (g == 0) {
    const float a = alpha ? *alpha : 1.0f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = wn * 64 + 32 * j + r;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int m = wm * 128 + 32 * i + 8 * (v / 4) + 4 * h + v % 4;
          const float sum = acc[i][j][v] + exchange[((p * 8 + i * 2 + j) * 16 + v) * L2C_WAVE + lane];
          // Nontemporal stores: 218.2-218.3 against 218.9-219.2 µs with
          // ordinary ones at 1024 x 16384 x 8192, one box.
          if (m < mrows && n < nrows)
            __builtin_nontemporal_store(sum * a, &out[static_cast<size_t>(m0 + m) * N + n0 + n]);
        }
    }
  }
}

}  // namespace

extern "C" int l2c_matmul_bf16(float *out, const uint16_t *X, const uint16_t *W, const float *alpha, int batch,
                               int cols, int rows, hipStream_t stream) {
  if (batch < 0 || cols <= 0 || rows < 0 || cols % 32 != 0) return hipErrorInvalidValue;
  if (batch == 0 || rows == 0) return hipSuccess;
  if (!out || !X || !W || !l2c_aligned16(X) || !l2c_aligned16(W)) return hipErrorInvalidValue;
  // The tile's operand windows stay addressable with 32-bit buffer offsets.
  if (static_cast<long long>(kBM) * cols * 2 > 0x7fffffffLL) return hipErrorInvalidValue;
  if (cols % 64 != 0) return l2c_matmul_bf16_split(out, X, W, alpha, batch, cols, rows, stream);
  const long long tiles = static_cast<long long>((batch + kBM - 1) / kBM) * ((rows + kBN - 1) / kBN);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(bf16_gemm_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, stream, out, X, W,
                     alpha, batch, rows, cols);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}
