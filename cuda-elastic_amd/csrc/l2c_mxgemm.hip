// MXFP6 x MXFP6 contraction on the gfx950 scaled matrix cores:
//   out[b][r] = sum_k deq(X)[b][k] * deq(W)[r][k],
// X and W both E3M2 codes with one UE8M0 scale byte per 32 values, in the
// tiled operand layout that l2c_quantize_mxfp6 writes. This is the classifier
// of the lowprec MXFP6 case (experiments/blackwell/lowprec/spec.json
// "cases.mxfp6", which runs CUTLASS's SM120 block-scaled GEMM; the arithmetic
// is the same: exact products of the dequantized operands, FP32 accumulation).
//
// Operand layout (rows padded to a multiple of 32; Rp = padded rows):
//   codes  [K / 128][Rp / 32][4 blocks][32 rows][24 B]  (24 B = 32 E3M2 codes,
//          the packed little-endian 6-bit stream of one 32-value block)
//   scales [K / 128][Rp][4 B]                          (byte b = block b)
// A tile's k-step slab (its rows' 4 blocks) is contiguous, and a lane's MFMA
// operand (one row, one block) is 24 contiguous bytes.
//
// Kernel design:
//  * v_mfma_scale_f32_32x32x64_f8f6f4 with both operands in format 3 (E3M2):
//    lane l supplies row l % 32 and one 32-value block in six VGPRs (its 24
//    packed bytes) plus that block's UE8M0 byte in a scale VGPR.
//  * Tile 256 (batch) x 128 (rows) x 128 (k per step), 8 wavefronts. Waves w and
//    w + 4 share a SIMD and the same 128 x 64 output sub-tile (4 x 2 blocks of
//    32 x 32); wave group g = w / 4 takes MFMA slice g of every step (lane half
//    h supplies block 2h + g). Per step each wave reads 9 KB of fragments:
//    72 KB per CU for 256 x 128 x 128 MACs, 25% less than 64 x 64 wave tiles,
//    at two waves per SIMD. The two groups' partial sums are added once at the
//    end through LDS, group 1's before group 0's in a fixed order.
//  * Staging by LDS DMA (buffer_load ... lds, 16 B a lane): each wave
//    instruction moves 1 KB of a slab straight into LDS with no VGPRs or
//    ds_write. 38 instructions a step over the 8 waves: X slab KB 8k + w
//    (k < 3), W slab KB w and 8 + w (w < 4), the X scale words (w = 4) and the W
//    scale words (w = 5). Three stages: step t's DMA is issued at step t - 2
//    and waited (vmcnt) before the barrier of step t - 1.
//  * Fragments: 3 x ds_read_b64 per operand. 32 lanes with consecutive rows
//    read 24-byte-strided data: 32 distinct even bank pairs, conflict free.
//  * Every access is in bounds by construction (no reliance on buffer range
//    checks): a tile's row groups past the operand's padded rows re-read its
//    last group (a wave-uniform clamp), and scale-word lanes past the padded
//    rows re-read its last four rows (a per-lane clamp). Those rows are
//    computed and never stored. K % 128 == 0.
//  * Workgroup order is remapped per XCD as in the other contractions.
#include "l2c_common.h"
#include "../../include/l2c.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_ptr;

constexpr int kBM = 256;
constexpr int kBN = 128;
constexpr int kThreads = 512;
constexpr int kStages = 3;
constexpr int kGroup = 4 * 32 * 24;           // one 32-row group per step: 3072 B
constexpr int kXBytes = (kBM / 32) * kGroup;  // 24 KB
constexpr int kWBytes = (kBN / 32) * kGroup;  // 12 KB
constexpr int kXS = kXBytes + kWBytes;        // X scale words: 256 x 4 B
constexpr int kWS = kXS + kBM * 4;            // W scale words: the DMA moves 256 x 4 B, 128 used
constexpr int kStage = kWS + 1024;
constexpr int kLds = kBM * kBN * 4;           // the partial-sum exchange; >= kStages * kStage
constexpr int kXcds = 8;
constexpr int kFmtE3M2 = 3;
static_assert(kStages * kStage <= kLds, "the stages fit the LDS allocation");

__global__ __launch_bounds__(kThreads, 1) void mxfp6_gemm_kernel(float *__restrict__ out,
                                                                 const uint8_t *__restrict__ X,
                                                                 const uint8_t *__restrict__ Xs,
                                                                 const uint8_t *__restrict__ W,
                                                                 const uint8_t *__restrict__ Ws, int M, int N,
                                                                 int K) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[kLds];
  int tile = blockIdx.x;
  const int tiles = gridDim.x;
  if (tiles % kXcds == 0) tile = (tile % kXcds) * (tiles / kXcds) + tile / kXcds;
  const int mtiles = (M + kBM - 1) / kBM;
  const int m0 = (tile % mtiles) * kBM, n0 = (tile / mtiles) * kBN;
  const int mrows = min(kBM, M - m0), nrows = min(kBN, N - n0);
  const int Mp = (M + 31) / 32 * 32, Np = (N + 31) / 32 * 32;
  const int tid = threadIdx.x, lane = tid % L2C_WAVE;
  const int wave = __builtin_amdgcn_readfirstlane(tid / L2C_WAVE);
  const int g = wave >> 2;                   // MFMA slice of this wave
  const int p = wave & 3;                    // output sub-tile
  const int wm = p & 1, wn = p >> 1;         // 128 x 64 at (128 wm, 64 wn)
  const int r = lane % 32, h = lane / 32;
  const int steps = K / 128;
  const int xstep = Mp / 32 * kGroup, wstep = Np / 32 * kGroup;
  const __amdgpu_buffer_rsrc_t rx = l2c::buffer_rsrc(X, static_cast<uint32_t>(xstep) * steps);
  const __amdgpu_buffer_rsrc_t rw = l2c::buffer_rsrc(W, static_cast<uint32_t>(wstep) * steps);
  const __amdgpu_buffer_rsrc_t rxs = l2c::buffer_rsrc(Xs, static_cast<uint32_t>(Mp) * 4 * steps);
  const __amdgpu_buffer_rsrc_t rws = l2c::buffer_rsrc(Ws, static_cast<uint32_t>(Np) * 4 * steps);
  const int lane16 = 16 * lane;
  // Slab KB d of a tile lies in its row group d / 3; groups past the padded
  // rows are replaced by the last one.
  const int xlast = Mp / 32 - 1 - m0 / 32, wlast = Np / 32 - 1 - n0 / 32;
  auto slab = [](int d, int glast) __attribute__((always_inline)) {
    return min(d / 3, glast) * kGroup + (d % 3) * 1024;
  };
  // Scale words: lane covers rows 4 lane .. 4 lane + 3 of the tile.
  const int xsl = min(lane16, (Mp - m0) * 4 - 16), wsl = min(lane16, (Np - n0) * 4 - 16);

  auto dma = [&](int stage, int t) __attribute__((always_inline)) {
    unsigned char *base = lds + stage * kStage;
    const int xs0 = xstep * t + (m0 / 32) * kGroup, ws0 = wstep * t + (n0 / 32) * kGroup;
#pragma unroll
    for (int k = 0; k < 3; ++k)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr *)(base + (8 * k + wave) * 1024), 16, lane16,
                                               xs0 + slab(8 * k + wave, xlast), 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr *)(base + kXBytes + wave * 1024), 16, lane16,
                                             ws0 + slab(wave, wlast), 0, 0);
    if (wave < 4)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr *)(base + kXBytes + (8 + wave) * 1024), 16, lane16,
                                               ws0 + slab(8 + wave, wlast), 0, 0);
    else if (wave == 4)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rxs, (lds_ptr *)(base + kXS), 16, xsl, Mp * 4 * t + m0 * 4, 0, 0);
    else if (wave == 5)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rws, (lds_ptr *)(base + kWS), 16, wsl, Np * 4 * t + n0 * 4, 0, 0);
  };
  // Waits for this wave's DMA of the older of two outstanding steps (waves
  // 0..5 issue 5 instructions a step, 6 and 7 issue 4) and its LDS reads, then
  // the workgroup barrier. Nothing is scheduled across it.
  auto sync = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    if (wave < 6)
      asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // Fragments: lane (r, h) supplies block blk = 2h + g of row r in group
  // wm * 4 + i (X, 3072 B apart) or wn * 2 + j (W).
  const int blk = 2 * h + g;
  const int shift = 8 * blk;
  const int ao = (wm * 16 + blk) * 768 + 24 * r;
  const int bo = kXBytes + (wn * 8 + blk) * 768 + 24 * r;
  const int sao = kXS + (wm * 128 + r) * 4;
  const int sbo = kWS + (wn * 64 + r) * 4;
  u32x2 fa[4][3], fb[2][3];
  unsigned sa[4], sb[2];
  auto read = [&](int stage) __attribute__((always_inline)) {
    const unsigned char *base = lds + stage * kStage;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int c = 0; c < 3; ++c) fa[i][c] = *reinterpret_cast<const u32x2 *>(base + ao + 3072 * i + 8 * c);
      sa[i] = *reinterpret_cast<const unsigned *>(base + sao + 128 * i) >> shift;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int c = 0; c < 3; ++c) fb[j][c] = *reinterpret_cast<const u32x2 *>(base + bo + 3072 * j + 8 * c);
      sb[j] = *reinterpret_cast<const unsigned *>(base + sbo + 128 * j) >> shift;
    }
  };
  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int last = steps - 1;
  dma(0, 0);
  dma(1, min(1, last));
  sync();  // step 0 landed
  read(0);
  int cur = 0;
  for (int t = 0; t < steps; ++t) {
    const int nxt = cur == kStages - 1 ? 0 : cur + 1;
    const int far = nxt == kStages - 1 ? 0 : nxt + 1;
    // Stage `far` was last read in step t - 1, before that step's barrier.
    dma(far, min(t + 2, last));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      i32x8 a;
      a[0] = fa[i][0][0], a[1] = fa[i][0][1], a[2] = fa[i][1][0], a[3] = fa[i][1][1];
      a[4] = fa[i][2][0], a[5] = fa[i][2][1], a[6] = 0, a[7] = 0;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        i32x8 b;
        b[0] = fb[j][0][0], b[1] = fb[j][0][1], b[2] = fb[j][1][0], b[3] = fb[j][1][1];
        b[4] = fb[j][2][0], b[5] = fb[j][2][1], b[6] = 0, b[7] = 0;
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc[i][j], kFmtE3M2, kFmtE3M2, 0,
                                                                     static_cast<int>(sa[i]), 0,
                                                                     static_cast<int>(sb[j]));
      }
    }
    sync();  // step t + 1 landed; every wave's reads of step t are done
    read(nxt);
    cur = nxt;
  }

  // Partial sums of the two slices: group 1 stores, group 0 adds and writes.
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
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = wn * 64 + 32 * j + r;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int m = wm * 128 + 32 * i + 8 * (v / 4) + 4 * h + v % 4;
          const float sum = acc[i][j][v] + exchange[((p * 8 + i * 2 + j) * 16 + v) * L2C_WAVE + lane];
          if (m < mrows && n < nrows) out[static_cast<size_t>(m0 + m) * N + n0 + n] = sum;
        }
    }
  }
}

}  // namespace

extern "C" int l2c_mxfp6_bytes(int rows, int width, size_t *code_bytes, size_t *scale_bytes) {
  if (rows < 0 || width <= 0 || width % 128 != 0 || !code_bytes || !scale_bytes) return hipErrorInvalidValue;
  const size_t padded = static_cast<size_t>((rows + 31) / 32) * 32;
  *code_bytes = padded * static_cast<size_t>(width) / 4 * 3;
  *scale_bytes = padded * static_cast<size_t>(width) / 32;
  return hipSuccess;
}

extern "C" int l2c_matmul_mxfp6(float *out, const uint8_t *X, const uint8_t *Xscales, const uint8_t *W,
                                const uint8_t *Wscales, int batch, int cols, int rows, hipStream_t stream) {
  if (batch < 0 || cols <= 0 || rows < 0 || cols % 128 != 0) return hipErrorInvalidValue;
  if (batch == 0 || rows == 0) return hipSuccess;
  if (!out || !X || !Xscales || !W || !Wscales || !l2c_aligned16(X) || !l2c_aligned16(W) ||
      !l2c_aligned16(Xscales) || !l2c_aligned16(Wscales))
    return hipErrorInvalidValue;
  // Whole operands stay addressable with the kernel's byte offsets, which it
  // computes in (signed) int.
  size_t xc, xs, wc, ws;
  l2c_mxfp6_bytes(batch, cols, &xc, &xs);
  l2c_mxfp6_bytes(rows, cols, &wc, &ws);
  if (xc > 0x7fffffffULL || wc > 0x7fffffffULL || xs > 0x7fffffffULL || ws > 0x7fffffffULL)
    return hipErrorInvalidValue;
  const long long tiles = static_cast<long long>((batch + kBM - 1) / kBM) * ((rows + kBN - 1) / kBN);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(mxfp6_gemm_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, stream, out, X,
                     Xscales, W, Wscales, batch, rows, cols);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}
