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
//    global memory with 16-byte buffer loads into registers while the previous
//    slab is multiplied out of LDS, then stored into the other half of a
//    double-buffered LDS ring: one barrier per step.
//  * Buffer loads: every lane's byte offset is computed once (rows past the
//    operand clamped to its last row) and the step offset k0 * 4 is a scalar,
//    so the main loop spends no vector instructions on addresses and has no
//    branches. A partial last step (K % 32 != 0) runs after the loop with
//    masked loads that fill zeros for k >= K.
//  * LDS rows keep the operands' K-contiguous layout with a row stride of
//    BK + 4 floats, so the 16-byte fragment reads of 16 consecutive lanes hit
//    64 distinct banks.
//  * MFMA operand layout: for v_mfma_f32_32x32x2f32 lane l supplies
//    A[l % 32][k = l / 32] and B[k = l / 32][l % 32]. Because the contraction
//    sums over k, the k index may be permuted as long as A and B use the same
//    permutation: lane l reads four consecutive k values (one ds_read_b128)
//    from k0 + 4 * (l / 32), and MFMA t of four consumes the t-th of them.
//    Four MFMAs therefore cover 8 consecutive k with one LDS read per operand.
//  * Instruction schedule of one step (four 8-deep k groups, 16 MFMAs each):
//    group g issues its global loads (g = 0) and the fragment reads of group
//    g + 1 ahead of its MFMAs, so LDS latency hides behind 16 MFMAs; the last
//    group interleaves the LDS stores of the next slab with its MFMAs.
//  * Accumulator layout of the 32 x 32 block: register v of lane l holds
//    C[8 * (v / 4) + 4 * (l / 32) + v % 4][l % 32].
//  * XCD-aware order: workgroup i is dispatched to XCD i % 8. The tile order
//    is remapped so that each XCD owns a contiguous band of N tiles (all M
//    tiles of those rows of W): every W slab is fetched from HBM into one L2,
//    and X (64 MiB at the large shape) is shared by the 32 CUs of an XCD.
//  * Operands whose rows are not 16-byte aligned (K % 4 != 0 or a misaligned
//    base pointer) take gemm_f32_generic_kernel: the same tiling with scalar,
//    bounds-checked loads.
#include "l2c_common.h"
#include "../../include/l2c.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
using l2c::f32x4;

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
constexpr int kGroups = kBK / 8;                         // 8-deep k groups per step
constexpr int kXcds = 8;
// The tile of one workgroup must stay addressable with the kernel's per-lane
// byte offsets, row * K * 4 computed in (signed) int; larger K takes the
// generic kernel, which indexes with size_t.
constexpr long long kMaxTileBytes = 0x7fffffffLL;

static_assert(kBM * kChunksPerRow % kThreads == 0, "A slab must split evenly");
static_assert(kBN * kChunksPerRow % kThreads == 0, "B slab must split evenly");
static_assert(kGroups == 4, "the instruction schedule below assumes four k groups per step");

// sched_group_barrier classes.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedVmemRead = 0x020;
constexpr int kSchedDsRead = 0x100;
constexpr int kSchedDsWrite = 0x200;

struct Smem {
  float a[2][kBM][kLdsStride];
  float b[2][kBN][kLdsStride];
};

__device__ __forceinline__ void tile_origin(int M, int &m0, int &n0) {
  int tile = blockIdx.x;
  const int tiles = gridDim.x;
  if (tiles % kXcds == 0) tile = (tile % kXcds) * (tiles / kXcds) + tile / kXcds;
  const int mtiles = (M + kBM - 1) / kBM;
  m0 = (tile % mtiles) * kBM;
  n0 = (tile / mtiles) * kBN;
}

__device__ __forceinline__ void zero_acc(f32x16 (&acc)[kFragM][kFragN]) {
#pragma unroll
  for (int i = 0; i < kFragM; ++i)
#pragma unroll
    for (int j = 0; j < kFragN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
}

// Lanes 0-31 and 32-63 each write 32 consecutive floats of an output row,
// with nontemporal stores (written once; 1848.7-1849.6 against 1850.8-1851.2
// µs with ordinary stores at 1024 x 16384 x 8192, one box).
__device__ __forceinline__ void store_tile(float *out, const f32x16 (&acc)[kFragM][kFragN], int m0,
                                           int n0, int M, int N, int wm, int wn, int lane) {
#pragma unroll
  for (int i = 0; i < kFragM; ++i) {
#pragma unroll
    for (int j = 0; j < kFragN; ++j) {
      const int n = n0 + wn * kWaveN + j * 32 + lane % 32;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * kWaveM + i * 32 + 8 * (v / 4) + 4 * (lane / 32) + v % 4;
        if (m < M && n < N) __builtin_nontemporal_store(acc[i][j][v], &out[static_cast<size_t>(m) * N + n]);
      }
    }
  }
}

// Fragment reads and MFMAs of one 8-deep k group, shared by both kernels.
struct Frags {
  f32x4 a[kFragM], b[kFragN];
};

__device__ __forceinline__ void read_frags(Frags &f, const float *a_base, const float *b_base,
                                           int buf, int kk) {
  constexpr int kABuf = kBM * kLdsStride, kBBuf = kBN * kLdsStride;
#pragma unroll
  for (int i = 0; i < kFragM; ++i)
    f.a[i] = *reinterpret_cast<const f32x4 *>(a_base + buf * kABuf + i * 32 * kLdsStride + kk);
#pragma unroll
  for (int j = 0; j < kFragN; ++j)
    f.b[j] = *reinterpret_cast<const f32x4 *>(b_base + buf * kBBuf + j * 32 * kLdsStride + kk);
}

__device__ __forceinline__ void mfma_group(f32x16 (&acc)[kFragM][kFragN], const Frags &f) {
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int i = 0; i < kFragM; ++i)
#pragma unroll
      for (int j = 0; j < kFragN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[i][c], f.b[j][c], acc[i][j], 0, 0, 0);
}

__global__ __launch_bounds__(kThreads) void gemm_f32_mfma_kernel(float *__restrict__ out,
                                                                 const float *__restrict__ X,
                                                                 const float *__restrict__ W,
                                                                 int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) Smem sm;
  int m0, n0;
  tile_origin(M, m0, n0);
  const int mrows = min(kBM, M - m0), nrows = min(kBN, N - n0);
  const int t = threadIdx.x;
  const int lane = t % L2C_WAVE;
  const int wave = t / L2C_WAVE;
  const int wm = wave % kWavesM;
  const int wn = wave / kWavesM;

  // Buffer resources over this tile's rows of X and W; per-lane byte offsets
  // of the slab chunks this thread stages (row clamped, k-step excluded).
  const __amdgpu_buffer_rsrc_t rx =
      l2c::buffer_rsrc(X + static_cast<size_t>(m0) * K, static_cast<uint32_t>(mrows) * K * 4u);
  const __amdgpu_buffer_rsrc_t rw =
      l2c::buffer_rsrc(W + static_cast<size_t>(n0) * K, static_cast<uint32_t>(nrows) * K * 4u);
  int xo[kLoadsA], wo[kLoadsB];
#pragma unroll
  for (int i = 0; i < kLoadsA; ++i) {
    const int idx = t + i * kThreads;
    xo[i] = min(idx / kChunksPerRow, mrows - 1) * K * 4 + (idx % kChunksPerRow) * 16;
  }
#pragma unroll
  for (int i = 0; i < kLoadsB; ++i) {
    const int idx = t + i * kThreads;
    wo[i] = min(idx / kChunksPerRow, nrows - 1) * K * 4 + (idx % kChunksPerRow) * 16;
  }

  f32x4 ga[kLoadsA], gb[kLoadsB];
  auto global_load = [&](int kt) __attribute__((always_inline)) {
    const int so = kt * kBK * 4;
#pragma unroll
    for (int i = 0; i < kLoadsA; ++i)
      ga[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, xo[i], so, 0));
#pragma unroll
    for (int i = 0; i < kLoadsB; ++i)
      gb[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo[i], so, 0));
  };
  // The partial last step: chunks at k >= K are zero in both operands.
  auto global_load_tail = [&](int kt) __attribute__((always_inline)) {
    const int so = kt * kBK * 4;
#pragma unroll
    for (int i = 0; i < kLoadsA; ++i) {
      const bool ok = kt * kBK + ((t + i * kThreads) % kChunksPerRow) * 4 < K;
      ga[i] = ok ? __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, xo[i], so, 0))
                 : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < kLoadsB; ++i) {
      const bool ok = kt * kBK + ((t + i * kThreads) % kChunksPerRow) * 4 < K;
      gb[i] = ok ? __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo[i], so, 0))
                 : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto lds_store = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kLoadsA; ++i) {
      const int idx = t + i * kThreads;
      *reinterpret_cast<f32x4 *>(&sm.a[buf][idx / kChunksPerRow][(idx % kChunksPerRow) * 4]) = ga[i];
    }
#pragma unroll
    for (int i = 0; i < kLoadsB; ++i) {
      const int idx = t + i * kThreads;
      *reinterpret_cast<f32x4 *>(&sm.b[buf][idx / kChunksPerRow][(idx % kChunksPerRow) * 4]) = gb[i];
    }
  };

  f32x16 acc[kFragM][kFragN];
  zero_acc(acc);
  const float *a_base = &sm.a[0][wm * kWaveM + lane % 32][4 * (lane / 32)];
  const float *b_base = &sm.b[0][wn * kWaveN + lane % 32][4 * (lane / 32)];
  Frags fr[2];

  const int nk = K / kBK;  // full steps
  if (nk > 0) {
    global_load(0);
    lds_store(0);
    __syncthreads();
    read_frags(fr[0], a_base, b_base, 0, 0);
    for (int kt = 0; kt < nk; ++kt) {
      const int buf = kt & 1;
      // The last step reloads itself: no branch, the stored copy is unused.
      global_load(min(kt + 1, nk - 1));
#pragma unroll
      for (int g = 0; g < kGroups; ++g) {
        if (g + 1 < kGroups) read_frags(fr[(g + 1) & 1], a_base, b_base, buf, (g + 1) * 8);
        mfma_group(acc, fr[g & 1]);
        if (g == kGroups - 1) lds_store(buf ^ 1);
        if (g == 0) {
          __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, kLoadsA + kLoadsB, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, kFragM + kFragN, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 16, 0);
        } else if (g + 1 < kGroups) {
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, kFragM + kFragN, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 16, 0);
        } else {
          for (int s = 0; s < kLoadsA + kLoadsB; ++s) {
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedDsWrite, 1, 0);
          }
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 16 - 2 * (kLoadsA + kLoadsB), 0);
        }
      }
      __syncthreads();
      read_frags(fr[0], a_base, b_base, buf ^ 1, 0);
    }
  }
  if (K % kBK != 0) {
    const int buf = nk & 1;
    __syncthreads();  // every wave is done with its last fragment reads
    global_load_tail(nk);
    lds_store(buf);
    __syncthreads();
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      read_frags(fr[0], a_base, b_base, buf, g * 8);
      mfma_group(acc, fr[0]);
    }
  }
  store_tile(out, acc, m0, n0, M, N, wm, wn, lane);
}

// Loads one float4 of a K-contiguous operand row with scalar, bounds-checked
// loads; zero outside [0, rows) x [0, K).
__device__ __forceinline__ f32x4 load_chunk_scalar(const float *base, int row, int rows, int k,
                                                   int K) {
  const bool row_ok = row < rows;
  const float *p = base + static_cast<size_t>(row_ok ? row : rows - 1) * K;
  f32x4 v;
  v[0] = row_ok && k < K ? p[k] : 0.f;
  v[1] = row_ok && k + 1 < K ? p[k + 1] : 0.f;
  v[2] = row_ok && k + 2 < K ? p[k + 2] : 0.f;
  v[3] = row_ok && k + 3 < K ? p[k + 3] : 0.f;
  return v;
}

// Any K and any 4-byte alignment: the tiling above with scalar loads and the
// compiler's own schedule.
__global__ __launch_bounds__(kThreads) void gemm_f32_generic_kernel(float *__restrict__ out,
                                                                    const float *__restrict__ X,
                                                                    const float *__restrict__ W,
                                                                    int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) Smem sm;
  int m0, n0;
  tile_origin(M, m0, n0);
  const int t = threadIdx.x;
  const int lane = t % L2C_WAVE;
  const int wave = t / L2C_WAVE;
  const int wm = wave % kWavesM;
  const int wn = wave / kWavesM;

  f32x4 ga[kLoadsA], gb[kLoadsB];
  auto global_load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < kLoadsA; ++i) {
      const int idx = t + i * kThreads;
      ga[i] = load_chunk_scalar(X, m0 + idx / kChunksPerRow, M, k0 + (idx % kChunksPerRow) * 4, K);
    }
#pragma unroll
    for (int i = 0; i < kLoadsB; ++i) {
      const int idx = t + i * kThreads;
      gb[i] = load_chunk_scalar(W, n0 + idx / kChunksPerRow, N, k0 + (idx % kChunksPerRow) * 4, K);
    }
  };
  auto lds_store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kLoadsA; ++i) {
      const int idx = t + i * kThreads;
      *reinterpret_cast<f32x4 *>(&sm.a[buf][idx / kChunksPerRow][(idx % kChunksPerRow) * 4]) = ga[i];
    }
#pragma unroll
    for (int i = 0; i < kLoadsB; ++i) {
      const int idx = t + i * kThreads;
      *reinterpret_cast<f32x4 *>(&sm.b[buf][idx / kChunksPerRow][(idx % kChunksPerRow) * 4]) = gb[i];
    }
  };

  f32x16 acc[kFragM][kFragN];
  zero_acc(acc);
  const float *a_base = &sm.a[0][wm * kWaveM + lane % 32][4 * (lane / 32)];
  const float *b_base = &sm.b[0][wn * kWaveN + lane % 32][4 * (lane / 32)];
  Frags fr[2];
  const int nk = (K + kBK - 1) / kBK;

  global_load(0);
  lds_store(0);
  __syncthreads();
  read_frags(fr[0], a_base, b_base, 0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) global_load((kt + 1) * kBK);
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      if (g + 1 < kGroups) read_frags(fr[(g + 1) & 1], a_base, b_base, buf, (g + 1) * 8);
      mfma_group(acc, fr[g & 1]);
    }
    if (more) lds_store(buf ^ 1);
    __syncthreads();
    if (more) read_frags(fr[0], a_base, b_base, buf ^ 1, 0);
  }
  store_tile(out, acc, m0, n0, M, N, wm, wn, lane);
}

// The buffer-load kernel needs 16-byte aligned rows and a tile that fits
// 32-bit byte offsets.
bool use_buffer_kernel(const float *X, const float *W, int cols) {
  return cols % 4 == 0 && l2c_aligned16(X) && l2c_aligned16(W) &&
         static_cast<long long>(kBM) * cols * 4 <= kMaxTileBytes;
}

}  // namespace

int l2c_gemm_launch_shape(int batch, int cols, int rows, int *grid, int *block,
                          int *blocks_per_cu) {
  *grid = ((batch + kBM - 1) / kBM) * ((rows + kBN - 1) / kBN);
  *block = kThreads;
  const void *fn = cols % 4 == 0 ? reinterpret_cast<const void *>(gemm_f32_mfma_kernel)
                                 : reinterpret_cast<const void *>(gemm_f32_generic_kernel);
  return static_cast<int>(hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, fn, kThreads, 0));
}

extern "C" int l2c_matmul(float *out, const float *X, const float *W, int batch, int cols,
                          int rows, hipStream_t stream) {
  // The generic kernel's k indexes (k + 3 of a 32-wide step) stay below INT_MAX.
  if (batch < 0 || cols <= 0 || cols > 0x7fffffff - kBK || rows < 0) return hipErrorInvalidValue;
  if (batch == 0 || rows == 0) return hipSuccess;
  if (!out || !X || !W) return hipErrorInvalidValue;
  const long long tiles =
      static_cast<long long>((batch + kBM - 1) / kBM) * ((rows + kBN - 1) / kBN);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(tiles)), block(kThreads);
  if (use_buffer_kernel(X, W, cols))
    hipLaunchKernelGGL(gemm_f32_mfma_kernel, grid, block, 0, stream, out, X, W, batch, rows, cols);
  else
    hipLaunchKernelGGL(gemm_f32_generic_kernel, grid, block, 0, stream, out, X, W, batch, rows,
                       cols);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}
