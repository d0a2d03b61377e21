// MXFP6 x MXFP6 contraction on the gfx950 scaled matrix cores:
//   out[b][r] = sum_k deq(X)[b][k] * deq(W)[r][k],
// X and W both E3M2 codes (packed 6-bit little-endian streams, 24 bytes per
// 32 values) with one UE8M0 scale byte per 32 values, [rows][K / 32]. This is
// the classifier of the lowprec MXFP6 case
// (experiments/blackwell/lowprec/spec.json "cases.mxfp6", which runs CUTLASS's
// SM120 block-scaled GEMM; the arithmetic is the same: exact products of the
// dequantized operands, FP32 accumulation).
//
// Kernel design:
//  * v_mfma_scale_f32_32x32x64_f8f6f4 with both operands in format 3 (E3M2):
//    lane l supplies row l % 32 and 32 consecutive k of one 32-value block in
//    six VGPRs, which are exactly the block's 24 packed bytes, plus that
//    block's UE8M0 scale in one byte of a scale VGPR. No conversion runs.
//  * A k-step is 128 values (4 blocks, 96 bytes per row). Lane half h of
//    MFMA slice s in {0, 1} supplies block 2h + s of the step, for both
//    operands, so a lane's data for the step are 48 contiguous bytes (blocks
//    2h and 2h + 1) and its scales are bytes 2h, 2h + 1 of the row's 4-byte
//    step word: the word shifted right by 16h, byte s chosen by op_sel.
//  * Tile 256 (batch) x 128 (rows) x 128 (k), 8 wavefronts of 64 x 64
//    (2 x 2 blocks of 32 x 32); a three-stage LDS ring, global loads four
//    steps ahead through two register sets, and the next step's fragments
//    read before each barrier (the schedule of the bf16-operand kernel in
//    l2c_qgemm.hip).
//  * LDS rows are 112 bytes (96 + 16 padding): 16 lanes reading the same
//    16-byte column of 16 consecutive rows hit 16 distinct bank groups.
//  * Buffer loads with clamped per-lane row offsets and the k-step in the
//    scalar offset; K % 128 == 0 (the lowprec cases require width % 128 == 0),
//    so there is no partial step. Rows past M or N load in-bounds data and are
//    never stored.
//  * Workgroup order is remapped per XCD as in the other contractions.
#include <type_traits>

#include "l2c_common.h"
#include "../../include/l2c.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBM = 256;
constexpr int kBN = 128;
constexpr int kBK = 128;                     // values per k-step
constexpr int kRowBytes = kBK * 6 / 8;       // 96 code bytes per row and step
constexpr int kStride = kRowBytes + 16;      // LDS row stride
constexpr int kWavesM = 4;
constexpr int kWavesN = 2;
constexpr int kThreads = kWavesM * kWavesN * L2C_WAVE;  // 512
constexpr int kFragM = kBM / kWavesM / 32;              // 2
constexpr int kFragN = kBN / kWavesN / 32;              // 2
constexpr int kStages = 3;
constexpr int kXcds = 8;
constexpr int kXChunks = kBM * kRowBytes / 16 / kThreads;  // 16-byte X chunks per thread: 3
constexpr int kWPieces = kBN * kRowBytes / 8 / kThreads;   // 8-byte W pieces per thread: 3
constexpr int kXBytes = kBM * kStride;
constexpr int kWBytes = kBN * kStride;
constexpr int kXScale = kXBytes + kWBytes;   // [256] step words of X scales
constexpr int kWScale = kXScale + kBM * 4;   // [128] step words of W scales
constexpr int kStage = kWScale + kBN * 4;
constexpr int kFmtE3M2 = 3;
static_assert(kXChunks * 16 * kThreads == kBM * kRowBytes, "X staging covers the tile");
static_assert(kWPieces * 8 * kThreads == kBN * kRowBytes, "W staging covers the tile");

__global__ __launch_bounds__(kThreads) void mxfp6_gemm_kernel(float *__restrict__ out,
                                                              const uint8_t *__restrict__ X,
                                                              const uint8_t *__restrict__ Xs,
                                                              const uint8_t *__restrict__ W,
                                                              const uint8_t *__restrict__ Ws,
                                                              int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kStages * kStage];

  int tile = blockIdx.x;
  const int tiles = gridDim.x;
  if (tiles % kXcds == 0) tile = (tile % kXcds) * (tiles / kXcds) + tile / kXcds;
  const int mtiles = (M + kBM - 1) / kBM;
  const int m0 = (tile % mtiles) * kBM;
  const int n0 = (tile / mtiles) * kBN;
  const int mrows = min(kBM, M - m0), nrows = min(kBN, N - n0);
  const int tid = threadIdx.x;
  const int lane = tid % L2C_WAVE;
  const int wave = tid / L2C_WAVE;
  const int wm = wave % kWavesM;
  const int wn = wave / kWavesM;
  const int r = lane % 32;
  const int h = lane / 32;

  const int row_bytes = K / 8 * 6;  // packed bytes per row
  const int srow_bytes = K / 32;    // scale bytes per row
  const __amdgpu_buffer_rsrc_t rx =
      l2c::buffer_rsrc(X + static_cast<size_t>(m0) * row_bytes, static_cast<uint32_t>(mrows) * row_bytes);
  const __amdgpu_buffer_rsrc_t rw =
      l2c::buffer_rsrc(W + static_cast<size_t>(n0) * row_bytes, static_cast<uint32_t>(nrows) * row_bytes);
  const __amdgpu_buffer_rsrc_t rxs =
      l2c::buffer_rsrc(Xs + static_cast<size_t>(m0) * srow_bytes, static_cast<uint32_t>(mrows) * srow_bytes);
  const __amdgpu_buffer_rsrc_t rws =
      l2c::buffer_rsrc(Ws + static_cast<size_t>(n0) * srow_bytes, static_cast<uint32_t>(nrows) * srow_bytes);

  // Staging assignments: global byte offsets without the step part and LDS
  // offsets within a stage.
  int xg[kXChunks], xs[kXChunks], wg[kWPieces], ws[kWPieces];
#pragma unroll
  for (int v = 0; v < kXChunks; ++v) {
    const int id = v * kThreads + tid, row = id / 6, c = id % 6;
    xg[v] = min(row, mrows - 1) * row_bytes + 16 * c;
    xs[v] = row * kStride + 16 * c;
  }
#pragma unroll
  for (int v = 0; v < kWPieces; ++v) {
    const int id = v * kThreads + tid, row = id / 12, c = id % 12;
    wg[v] = min(row, nrows - 1) * row_bytes + 8 * c;
    ws[v] = kXBytes + row * kStride + 8 * c;
  }
  // Scale words: threads 0..255 stage X rows, 256..511 stage W rows (twice
  // over, the same word to the same slot).
  const bool sx = tid < kBM;
  const int srow = sx ? tid : (tid - kBM) % kBN;
  const int sg = min(srow, (sx ? mrows : nrows) - 1) * srow_bytes;
  const int ss = (sx ? kXScale : kWScale) + 4 * srow;

  u32x4 gx[2][kXChunks];
  u32x2 gw[2][kWPieces];
  unsigned gs[2];
  auto gload = [&](auto set, int t) __attribute__((always_inline)) {
    constexpr int st = decltype(set)::value;
#pragma unroll
    for (int v = 0; v < kXChunks; ++v) gx[st][v] = __builtin_amdgcn_raw_buffer_load_b128(rx, xg[v], kRowBytes * t, 0);
#pragma unroll
    for (int v = 0; v < kWPieces; ++v) gw[st][v] = __builtin_amdgcn_raw_buffer_load_b64(rw, wg[v], kRowBytes * t, 0);
    gs[st] = sx ? __builtin_amdgcn_raw_buffer_load_b32(rxs, sg, 4 * t, 0)
                : __builtin_amdgcn_raw_buffer_load_b32(rws, sg, 4 * t, 0);
  };
  auto lstore = [&](auto set, int stage) __attribute__((always_inline)) {
    constexpr int st = decltype(set)::value;
    unsigned char *base = lds + stage * kStage;
#pragma unroll
    for (int v = 0; v < kXChunks; ++v) *reinterpret_cast<u32x4 *>(base + xs[v]) = gx[st][v];
#pragma unroll
    for (int v = 0; v < kWPieces; ++v) *reinterpret_cast<u32x2 *>(base + ws[v]) = gw[st][v];
    *reinterpret_cast<unsigned *>(base + ss) = gs[st];
  };

  f32x16 acc[kFragM][kFragN];
#pragma unroll
  for (int i = 0; i < kFragM; ++i)
#pragma unroll
    for (int j = 0; j < kFragN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // This lane's fragments: X rows wm * 64 + 32 i + r, W rows wn * 64 + 32 j + r,
  // bytes 48h .. 48h + 47 of the step.
  const int arow = wm * kFragM * 32 + r;
  const int brow = wn * kFragN * 32 + r;
  struct Frags {
    u32x4 a[kFragM][3];
    u32x4 b[kFragN][3];
    unsigned sa[kFragM], sb[kFragN];
  };
  auto read_frags = [&](int stage, Frags &f) __attribute__((always_inline)) {
    const unsigned char *base = lds + stage * kStage;
#pragma unroll
    for (int i = 0; i < kFragM; ++i) {
#pragma unroll
      for (int c = 0; c < 3; ++c)
        f.a[i][c] = *reinterpret_cast<const u32x4 *>(base + (arow + 32 * i) * kStride + 48 * h + 16 * c);
      f.sa[i] = *reinterpret_cast<const unsigned *>(base + kXScale + 4 * (arow + 32 * i)) >> (16 * h);
    }
#pragma unroll
    for (int j = 0; j < kFragN; ++j) {
#pragma unroll
      for (int c = 0; c < 3; ++c)
        f.b[j][c] = *reinterpret_cast<const u32x4 *>(base + kXBytes + (brow + 32 * j) * kStride + 48 * h + 16 * c);
      f.sb[j] = *reinterpret_cast<const unsigned *>(base + kWScale + 4 * (brow + 32 * j)) >> (16 * h);
    }
  };
  // Slice s: dwords 6s .. 6s + 5 of the lane's 12 (block 2h + s).
  auto operand = [](const u32x4 (&q)[3], int s) __attribute__((always_inline)) {
    i32x8 o;
    if (s == 0) {
      o[0] = q[0][0], o[1] = q[0][1], o[2] = q[0][2], o[3] = q[0][3], o[4] = q[1][0], o[5] = q[1][1];
    } else {
      o[0] = q[1][2], o[1] = q[1][3], o[2] = q[2][0], o[3] = q[2][1], o[4] = q[2][2], o[5] = q[2][3];
    }
    o[6] = 0, o[7] = 0;
    return o;
  };
  auto mma = [&](const Frags &f) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kFragM; ++i)
#pragma unroll
      for (int j = 0; j < kFragN; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(operand(f.a[i], 0), operand(f.b[j], 0),
                                                                     acc[i][j], kFmtE3M2, kFmtE3M2, 0,
                                                                     static_cast<int>(f.sa[i]), 0,
                                                                     static_cast<int>(f.sb[j]));
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(operand(f.a[i], 1), operand(f.b[j], 1),
                                                                     acc[i][j], kFmtE3M2, kFmtE3M2, 1,
                                                                     static_cast<int>(f.sa[i]), 1,
                                                                     static_cast<int>(f.sb[j]));
      }
  };

  Frags fr[2];
  const int steps = K / kBK;
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  // Steps past the last are clamped to it: redundant in-bounds loads whose
  // copies are never read.
  const int last = steps - 1;
  gload(I0(), 0);
  gload(I1(), min(1, last));
  lstore(I0(), 0);
  gload(I0(), min(2, last));
  lstore(I1(), 1);
  gload(I1(), min(3, last));
  __syncthreads();
  read_frags(0, fr[0]);
  int rd = 0;  // stage of the current step
  int t = 0;
  auto step = [&](auto set) __attribute__((always_inline)) {
    constexpr int st = decltype(set)::value;
    const int nx = rd == kStages - 1 ? 0 : rd + 1;
    const int wr = rd == 0 ? kStages - 1 : rd - 1;
    read_frags(nx, fr[st ^ 1]);
    mma(fr[st]);
    lstore(set, wr);
    gload(set, min(t + 4, last));
    __syncthreads();
    rd = nx;
    ++t;
  };
  for (; t + 2 <= steps;) {
    step(I0());
    step(I1());
  }
  if (t < steps) mma(fr[0]);

#pragma unroll
  for (int j = 0; j < kFragN; ++j) {
    const int n = brow + 32 * j;
#pragma unroll
    for (int i = 0; i < kFragM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = wm * kFragM * 32 + 32 * i + 8 * (v / 4) + 4 * h + v % 4;
        if (m < mrows && n < nrows) out[static_cast<size_t>(m0 + m) * N + n0 + n] = acc[i][j][v];
      }
    }
  }
}

}  // namespace

extern "C" int l2c_matmul_mxfp6(float *out, const uint8_t *X, const uint8_t *Xscales, const uint8_t *W,
                                const uint8_t *Wscales, int batch, int cols, int rows, hipStream_t stream) {
  if (batch < 0 || cols <= 0 || rows < 0 || cols % kBK != 0) return hipErrorInvalidValue;
  if (batch == 0 || rows == 0) return hipSuccess;
  if (!out || !X || !Xscales || !W || !Wscales || !l2c_aligned16(X) || !l2c_aligned16(W) ||
      (reinterpret_cast<uintptr_t>(Xscales) & 3u) || (reinterpret_cast<uintptr_t>(Wscales) & 3u))
    return hipErrorInvalidValue;
  // Per-workgroup operand windows stay addressable with 32-bit offsets.
  if (static_cast<long long>(kBM) * (cols / 8 * 6) > 0x7fffffffLL) return hipErrorInvalidValue;
  const long long tiles = static_cast<long long>((batch + kBM - 1) / kBM) * ((rows + kBN - 1) / kBN);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(mxfp6_gemm_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, stream, out, X,
                     Xscales, W, Wscales, batch, rows, cols);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}
