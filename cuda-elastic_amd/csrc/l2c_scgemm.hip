// Block-scaled quantized-weight contraction on the gfx950 scaled matrix cores:
//   out[b][r] = sum_k deq(Xq)[b][k] * deq(W)[r][k],
// where Xq is the bf16 activations quantized on the device to MXFP8 (E4M3
// codes, one UE8M0 scale per 32 k) and W the same quantized weights that
// l2c_matmul_q takes: MXFP4 (E2M1 codes, UE8M0 scale per 32 k) or E4M3 codes
// with one fp32 scale per row. The products are exact; accumulation is the
// matrix core's FP32.
//
// Activation quantizer (HBM bound; per element 2 B read, 1 B + 1/32 B
// written): one lane per 8 consecutive values (one 16-byte load), four lanes
// per 32-value block, the block maximum reduced across the four lanes. The
// shared exponent is the smallest X with amax <= 448 * 2^X, read off amax's
// fields: floor(log2 amax) - 8, plus one when amax's significand exceeds
// 1.75 (448 = 1.75 * 2^8), clamped below at -127; elements are
// E4M3(v * 2^-X), nearest-even, never beyond 448, by the hardware conversion
// (v_cvt_pk_fp8_f32) with negative zeros written as +0; its codes equal
// l2c_formats.h e4m3_code's (tested exhaustively against the oracle). The
// software encoder took ~40 VALU instructions a value and made the kernel
// VALU bound (17.7 us against ~7 us of HBM time at 1024 x 16384).
// Workspace layout: codes row-major [batch][cols]; at offset
// round_up(batch * cols, 256) the scales in k-step tiles [cols / 128][Bp][4]
// (Bp = batch rounded up to 4; byte j of a row's word is block j of the
// 128-k step; padding rows hold 0), so one step's scale words of a 256-row
// tile are 1 KB contiguous.
//
// Contraction kernel:
//  * v_mfma_scale_f32_32x32x64_f8f6f4, A = activations in format 0 (E4M3,
//    8 VGPRs a lane: 32 codes), B = weights in format 4 (E2M1, 4 VGPRs: 32
//    codes) or 0 (E4M3). Lane l supplies row l % 32 of its operand; lane half
//    h = l / 32 supplies the scale byte of the instruction's k-block
//    [32 h, 32 h + 32). Where each code sits in k differs by format
//    (measured on MI355X, operands and outputs fitted against the oracle's
//    arithmetic; only this placement fits, to fp32 rounding): an E2M1
//    operand's half h holds k [32 h, 32 h + 32) in order; an E4M3 operand's
//    half h holds k [16 h, 16 h + 16) in VGPRs 0-3 and k [32 + 16 h,
//    32 + 16 h + 16) in VGPRs 4-7. So an E4M3 lane takes the h-th 16-value
//    half of each of the instruction's two blocks, an E2M1 lane one whole
//    block. The fp8 weights' block scale is 2^0; their fp32 row scale
//    multiplies the output.
//  * Tile 256 (batch) x 128 (rows) x 128 (k per step), 8 wavefronts. Waves w
//    and w + 4 share a SIMD and a 128 x 64 output sub-tile (4 x 2 blocks of
//    32 x 32); wave group g = w / 4 takes the MFMA k-slice [64 g, 64 g + 64)
//    of every step, lane half h block 2 g + h. The two groups' partial sums
//    are added once at the end through LDS, group 1's before group 0's.
//  * Staging by LDS DMA (buffer_load ... lds, 16 B a lane) from the row-major
//    operands: X codes 32 KB a step (32 one-KB instructions, 8 rows of 128 B
//    each), the X scale words (one instruction), W codes 8 KB (MXFP4, 16 rows
//    of 64 B an instruction) or 16 KB (fp8), MXFP4 W scales as 4-byte DMAs,
//    one row a lane. 16-byte chunks of LDS rows are XOR-swizzled by row bits
//    (128-byte rows: bits 1..3; 64-byte rows: bits 2..3), applied on the
//    DMA's source side, so 32 lanes reading one chunk of 32 consecutive rows
//    hit distinct bank groups. Three stages (124 KB MXFP4, 147 KB fp8) on a
//    ping-pong schedule: the two waves of a SIMD alternate a memory phase
//    (DMA issue, fragment reads, DMA wait) and an MFMA phase half a step
//    apart, so the matrix core runs one wave's MFMAs while the other reads
//    LDS (details at the loop).
//  * Every access is in bounds by construction: operand rows past the end are
//    clamped per lane to the last row, scale words past the padded rows to
//    the last four rows; those rows are computed and never stored.
//  * Workgroup order is remapped per XCD as in the other contractions.
#include <mutex>

#include "l2c_common.h"
#include "l2c_formats.h"
#include "../../include/l2c.h"

// Fixed scratch of l2c_matmul_qs_static: the MXFP8 activations of one call.
// Each GPU the library runs on holds its own copy until the process ends.
// In host code `scratch` is only a stand-in for the symbol: its device
// address comes from hipGetSymbolAddress (per device, below), and only that
// address is passed to kernels.
static __device__ __align__(256) uint8_t scratch[L2C_QS_STATIC_SCRATCH_BYTES];

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_ptr;

constexpr int kBM = 256;
constexpr int kBN = 128;
constexpr int kBK = 128;
constexpr int kThreads = 512;
constexpr int kStages = 3;
constexpr int kXcds = 8;
constexpr int kFmtE4M3 = 0;
constexpr int kFmtE2M1 = 4;
constexpr int kExchange = 131072;  // 4 sub-tiles x 8 blocks x 16 values x 64 lanes x 4 B

size_t round256(size_t n) { return (n + 255) / 256 * 256; }
__host__ __device__ __forceinline__ int padded4(int rows) { return (rows + 3) / 4 * 4; }

template <int FMT>
struct Geometry {
  static constexpr bool kMx = FMT == L2C_Q_MXFP4;
  static constexpr int kXBytes = kBM * kBK;      // 32 KB of X codes
  static constexpr int kWRow = kMx ? 64 : 128;   // W code bytes per row and step
  static constexpr int kWBytes = kBN * kWRow;
  static constexpr int kXS = kXBytes + kWBytes;  // X scale words, 256 x 4 B
  static constexpr int kWS = kXS + kBM * 4;      // W scale words, 128 x 4 B (MXFP4)
  static constexpr int kStage = kWS + (kMx ? kBN * 4 : 0);
  static constexpr int kLds = kStages * kStage > kExchange ? kStages * kStage : kExchange;
  // DMA instructions a wave issues per step: X codes 4, W codes 1 (MXFP4) or
  // 2 (fp8), plus the X scales on wave 4 and the W scales on waves 5 and 6.
  static __device__ __forceinline__ int dma_count(int wave) {
    return 4 + (kMx ? 1 : 2) + (wave == 4 ? 1 : 0) + (kMx && (wave == 5 || wave == 6) ? 1 : 0);
  }
  static __device__ __forceinline__ int wswizzle(int row) { return kMx ? (row >> 2) & 3 : (row >> 1) & 7; }
};
static_assert(kStages * Geometry<L2C_Q_FP8>::kStage <= 160 * 1024, "the fp8 stages fit the LDS");

__device__ __forceinline__ int xswizzle(int row) { return (row >> 1) & 7; }

// ---------------------------------------------------------------------------
// Activation quantizer.

constexpr int kQuantChunks = 4;  // 16-byte chunks a thread converts

// Workgroup (x, y) converts chunks [1024 x, 1024 x + 1024) of rows y,
// y + gridDim.y, ... (a row is cols / 8 chunks of 8 values); thread t takes
// chunks t + 256 u (u < 4) of the segment, all four loads issued before any is
// used. Four consecutive chunks are one 32-value block (their maxima reduced
// by shuffles), sixteen one 128-k step, whose four scale bytes the step's
// first lane gathers by shuffles and stores as one word. Every lane runs every
// shuffle; only the loads and stores are predicated. Rows past `rows` (up to
// the scale tiles' padding) write zero scale words and no codes.
__global__ __launch_bounds__(256) void quantize_mxfp8_kernel(uint8_t *__restrict__ codes,
                                                             uint8_t *__restrict__ scales,
                                                             const uint16_t *__restrict__ X, int rows,
                                                             int rows_padded, int cols) {
  const int lanes_per_row = cols / 8;  // a multiple of 16 (cols % 128 == 0)
  const int first = blockIdx.x * (256 * kQuantChunks) + threadIdx.x;
  for (int row = blockIdx.y; row < rows_padded; row += gridDim.y) {
    const bool live_row = row < rows;
    const uint16_t *src = X + static_cast<size_t>(row) * cols;
    u32x4 raw[kQuantChunks];
#pragma unroll
    for (int u = 0; u < kQuantChunks; ++u) {
      const int chunk = first + 256 * u;
      raw[u] = u32x4{0u, 0u, 0u, 0u};
      if (live_row && chunk < lanes_per_row) raw[u] = *reinterpret_cast<const u32x4 *>(src + 8 * chunk);
    }
#pragma unroll
    for (int u = 0; u < kQuantChunks; ++u) {
      const int chunk = first + 256 * u;
      float v[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(raw[u][i] << 16);
        v[2 * i + 1] = __uint_as_float(raw[u][i] & 0xffff0000u);
      }
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
      amax = fmaxf(amax, __shfl_xor(amax, 1));
      amax = fmaxf(amax, __shfl_xor(amax, 2));
      // ceil(log2(amax / 448)): the exponent field less 127 + 8, plus one above
      // a significand of 1.75 (mantissa field 0x600000); a zero or subnormal
      // maximum clamps to -127, and the largest field, 254, gives at most 120.
      const unsigned abits = __float_as_uint(amax);
      const int x =
          max(static_cast<int>((abits >> 23) & 0xffu) - 135 + ((abits & 0x7fffffu) > 0x600000u ? 1 : 0), -127);
      const float inv = __uint_as_float(static_cast<unsigned>(127 - x) << 23);  // 2^-x, exact
      // E4M3 codes by the hardware conversion (nearest-even; |v * inv| <= 448,
      // so it never saturates), then negative zeros, which it keeps, made +0.
      unsigned packed[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        int w = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * h] * inv, v[4 * h + 1] * inv, 0, false);
        w = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * h + 2] * inv, v[4 * h + 3] * inv, w, true);
        const unsigned c = static_cast<unsigned>(w);
        const unsigned nonzero = ((c & 0x7f7f7f7fu) + 0x7f7f7f7fu) & 0x80808080u;  // 0x80 where magnitude != 0
        packed[h] = c & (nonzero | 0x7f7f7f7fu);
      }
      // The step's four block scales, from chunks 0, 4, 8 and 12 of its 16.
      const unsigned sbyte = live_row ? static_cast<unsigned>(x + 127) : 0u;
      const unsigned word = sbyte | (__shfl_down(sbyte, 4, 16) << 8) | (__shfl_down(sbyte, 8, 16) << 16) |
                            (__shfl_down(sbyte, 12, 16) << 24);
      if (live_row && chunk < lanes_per_row)
        *reinterpret_cast<uint2 *>(codes + static_cast<size_t>(row) * cols + 8 * chunk) =
            make_uint2(packed[0], packed[1]);
      if (chunk < lanes_per_row && (chunk & 15) == 0)
        *reinterpret_cast<unsigned *>(scales + (static_cast<size_t>(chunk / 16) * rows_padded + row) * 4) = word;
    }
  }
}

// ---------------------------------------------------------------------------
// The contraction.

template <int FMT>
__global__ __launch_bounds__(kThreads, 1) void scaled_gemm_kernel(float *__restrict__ out,
                                                                  const uint8_t *__restrict__ Xc,
                                                                  const uint8_t *__restrict__ Xs,
                                                                  const uint8_t *__restrict__ Wq,
                                                                  const void *__restrict__ wscales, int M,
                                                                  int N, int K) {
  using G = Geometry<FMT>;
  __shared__ __attribute__((aligned(1024))) unsigned char lds[G::kLds];
  int tile = blockIdx.x;
  const int tiles = gridDim.x;
  if (tiles % kXcds == 0) tile = (tile % kXcds) * (tiles / kXcds) + tile / kXcds;
  const int mtiles = (M + kBM - 1) / kBM;
  const int m0 = (tile % mtiles) * kBM, n0 = (tile / mtiles) * kBN;
  const int mrows = min(kBM, M - m0), nrows = min(kBN, N - n0);
  const int Mp = padded4(M);
  const int tid = threadIdx.x, lane = tid % L2C_WAVE;
  const int wave = __builtin_amdgcn_readfirstlane(tid / L2C_WAVE);
  const int g = wave >> 2, p = wave & 3;
  const int wm = p & 1, wn = p >> 1;
  const int r = lane % 32, h = lane / 32;
  const int steps = K / kBK;
  const int wrb = G::kMx ? K / 2 : K;  // W code bytes per row
  const int srb = K / 32;              // MXFP4 W scale bytes per row
  const __amdgpu_buffer_rsrc_t rx =
      l2c::buffer_rsrc(Xc + static_cast<size_t>(m0) * K, static_cast<uint32_t>(mrows) * K);
  const __amdgpu_buffer_rsrc_t rxs = l2c::buffer_rsrc(Xs, static_cast<uint32_t>(Mp) * 4 * steps);
  const __amdgpu_buffer_rsrc_t rw =
      l2c::buffer_rsrc(Wq + static_cast<size_t>(n0) * wrb, static_cast<uint32_t>(nrows) * wrb);
  const __amdgpu_buffer_rsrc_t rws =
      G::kMx ? l2c::buffer_rsrc(static_cast<const uint8_t *>(wscales) + static_cast<size_t>(n0) * srb,
                                static_cast<uint32_t>(nrows) * srb)
             : rw;

  // Per-lane DMA sources (the step's k offset is scalar). X: instruction
  // 8k + wave (k < 4) fills rows 8 (8k + wave) + lane / 8, slot lane % 8 with
  // chunk slot ^ xswizzle(row). W (MXFP4): instruction `wave` fills rows
  // 16 wave + lane / 4, slot lane % 4; W (fp8): instructions 8k + wave (k < 2)
  // as X. X scales (wave 4): lane covers rows 4 lane .. 4 lane + 3. W scales
  // (waves 5, 6): row 64 (wave - 5) + lane.
  int xsrc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int row = 8 * (8 * k + wave) + lane / 8;
    xsrc[k] = min(row, mrows - 1) * K + 16 * ((lane % 8) ^ xswizzle(row));
  }
  int wsrc[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if constexpr (G::kMx) {
      const int row = 16 * wave + lane / 4;
      wsrc[k] = min(row, nrows - 1) * wrb + 16 * ((lane % 4) ^ G::wswizzle(row));
    } else {
      const int row = 8 * (8 * k + wave) + lane / 8;
      wsrc[k] = min(row, nrows - 1) * wrb + 16 * ((lane % 8) ^ G::wswizzle(row));
    }
  }
  const int xssrc = min(16 * lane, (Mp - m0) * 4 - 16);
  const int wssrc = min(64 * max(wave - 5, 0) + lane, nrows - 1) * srb;

  auto dma = [&](int stage, int t) __attribute__((always_inline)) {
    unsigned char *base = lds + stage * G::kStage;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr *)(base + (8 * k + wave) * 1024), 16, xsrc[k], kBK * t,
                                               0, 0);
    if constexpr (G::kMx) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr *)(base + G::kXBytes + wave * 1024), 16, wsrc[0],
                                               64 * t, 0, 0);
      if (wave == 5 || wave == 6)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rws, (lds_ptr *)(base + G::kWS + (wave - 5) * 256), 4, wssrc,
                                                 4 * t, 0, 0);
    } else {
#pragma unroll
      for (int k = 0; k < 2; ++k)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr *)(base + G::kXBytes + (8 * k + wave) * 1024), 16,
                                                 wsrc[k], kBK * t, 0, 0);
    }
    if (wave == 4)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rxs, (lds_ptr *)(base + G::kXS), 16, xssrc, Mp * 4 * t + m0 * 4, 0,
                                               0);
  };
  // This wave's DMA of the older of two outstanding steps has landed and its
  // LDS reads are done; then the workgroup barrier. Nothing is scheduled
  // across it.
  const int outstanding = G::dma_count(wave);
  auto wait_dma_barrier = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    if (outstanding == 5)
      asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else if (outstanding == 6)
      asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(7) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  auto barrier = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // Fragments of lane (r, h) for the instruction over the step's blocks
  // 2 g and 2 g + 1 (16-byte chunks 4 g .. 4 g + 3 of a 128-byte fp8 row,
  // chunks 2 g, 2 g + 1 of a 64-byte MXFP4 row): X rows wm * 128 + 32 i + r,
  // chunks 4 g + h and 4 g + 2 + h (the h-th halves of both blocks); W rows
  // wn * 64 + 32 j + r, fp8 the same two chunks, MXFP4 chunk 2 g + h (block
  // 2 g + h whole). Scale bytes: block 2 g + h of the row's word for both
  // operands. The swizzle of row + 32 equals that of row.
  const int blk = 2 * g + h;
  const int xsw = xswizzle(r);
  const int xa = (wm * 128 + r) * 128;
  const int xc0 = 16 * ((4 * g + h) ^ xsw), xc1 = 16 * ((4 * g + 2 + h) ^ xsw);
  const int wr0 = wn * 64 + r;
  const int wsw = G::wswizzle(wr0);
  const int wa = G::kXBytes + wr0 * G::kWRow;
  const int wc0 = G::kMx ? 16 * (blk ^ wsw) : 16 * ((4 * g + h) ^ wsw);
  const int wc1 = 16 * ((4 * g + 2 + h) ^ wsw);
  const int shift = 8 * blk;
  u32x4 fa[4][2], fb[2][2];
  unsigned sa[4], sb[2];
  auto read = [&](int stage) __attribute__((always_inline)) {
    const unsigned char *base = lds + stage * G::kStage;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[i][0] = *reinterpret_cast<const u32x4 *>(base + xa + 4096 * i + xc0);
      fa[i][1] = *reinterpret_cast<const u32x4 *>(base + xa + 4096 * i + xc1);
      sa[i] = *reinterpret_cast<const unsigned *>(base + G::kXS + (wm * 128 + 32 * i + r) * 4) >> shift;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      fb[j][0] = *reinterpret_cast<const u32x4 *>(base + wa + 32 * G::kWRow * j + wc0);
      if constexpr (G::kMx)
        sb[j] = *reinterpret_cast<const unsigned *>(base + G::kWS + (wr0 + 32 * j) * 4) >> shift;
      else
        fb[j][1] = *reinterpret_cast<const u32x4 *>(base + wa + 32 * G::kWRow * j + wc1);
    }
  };
  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // Ping-pong schedule: the two waves of a SIMD (one per group) run half a step
  // apart. In its memory phase of step t a wave issues its DMA of step t + 2
  // into the stage step t - 1 held and reads its fragments of step t (in the
  // order below), and waits for its own DMA of step t + 1; in its MFMA phase it
  // runs its 8 MFMAs of step t at raised priority. Group 0's memory phase of
  // step t runs beside group 1's MFMA phase of step t - 1, and a workgroup
  // barrier ends every phase. Why three stages suffice: a stage is refilled in
  // the memory phase after the last one that read it (both groups read step t -
  // 1 before group 0's memory phase of step t begins), and a step's data has
  // landed everywhere one memory phase before its first reader, because each
  // wave waits for its own DMA one step ahead. Group 1 passes one extra barrier
  // at the start and group 0 one at the end, so both pass the same number.
  const int last = steps - 1;
  dma(0, 0);
  dma(1, min(1, last));
  wait_dma_barrier();  // step 0 landed everywhere
  if (g == 1) barrier();
  int cur = 0;
  for (int t = 0; t < steps; ++t) {
    // The order of the DMA issue and the fragment reads: each order measured
    // 2-2.6% faster for one format (MXFP4 114.1-114.8 against 117.0-117.3 µs
    // with the DMA first; fp8 125.3-125.9 against 127.9-128.1 µs with the
    // reads first, at 1024 x 16384 x 8192).
    if constexpr (G::kMx) {
      dma(cur == 0 ? kStages - 1 : cur - 1, min(t + 2, last));
      read(cur);
    } else {
      read(cur);
      dma(cur == 0 ? kStages - 1 : cur - 1, min(t + 2, last));
    }
    wait_dma_barrier();
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      i32x8 a;
#pragma unroll
      for (int c = 0; c < 4; ++c) a[c] = static_cast<int>(fa[i][0][c]), a[4 + c] = static_cast<int>(fa[i][1][c]);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        i32x8 b;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          b[c] = static_cast<int>(fb[j][0][c]);
          b[4 + c] = G::kMx ? 0 : static_cast<int>(fb[j][1][c]);
        }
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            a, b, acc[i][j], kFmtE4M3, G::kMx ? kFmtE2M1 : kFmtE4M3, 0, static_cast<int>(sa[i]), 0,
            G::kMx ? static_cast<int>(sb[j]) : 127);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    barrier();
    cur = cur == kStages - 1 ? 0 : cur + 1;
  }
  if (g == 0) barrier();

  // Partial sums of the two k-slices: group 1 stores, group 0 adds and writes.
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
      float rscale = 1.0f;
      if constexpr (!G::kMx) rscale = n < nrows ? static_cast<const float *>(wscales)[n0 + n] : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int m = wm * 128 + 32 * i + 8 * (v / 4) + 4 * h + v % 4;
          const float sum = acc[i][j][v] + exchange[((p * 8 + i * 2 + j) * 16 + v) * L2C_WAVE + lane];
          // Nontemporal stores: MXFP4 112.5-112.8 against 114.1-114.3 µs with
          // ordinary ones, fp8 123.2-123.7 against 125.3-125.5 (the product,
          // quantizer included, at 1024 x 16384 x 8192 on one box).
          if (m < mrows && n < nrows)
            __builtin_nontemporal_store(sum * rscale, &out[static_cast<size_t>(m0 + m) * N + n0 + n]);
        }
    }
  }
}

// ---------------------------------------------------------------------------
// The MXFP4 contraction on wide tiles: 128 (batch) x 256 (rows) x 128 (k per
// step). Both operands are staged by LDS DMA from L2, and the L2 serves a
// request per row segment whatever its length up to a 128-byte line, so the
// staging time tracks the number of row segments rather than the bytes. X
// codes are 128 bytes a row and step (one line); the E2M1 W codes are only 64,
// so W is staged two steps at a time: 256 rows x 128 bytes (steps 2 p and
// 2 p + 1, 32 one-KB instructions, 4 a wave) into one of two pair slots every
// other step. Per two steps that is 256 + 256 row segments against 256 + 512
// with W staged a step at a time, at the same instruction count; a
// staging-only copy of the two patterns (`l2c_kernel_bench stage_wpair` and
// `stage_wstep`) measured 42.6 against 58.6 µs at 1024 x 16384 x 8192, the
// kernel 106.9 against 108.0 µs (1%; the C5 graph iteration 136.4-137.8
// against 138.4-139.8), results bit-identical. The W scales are staged 16
// bytes a row, the scale words of four
// consecutive steps (row-major [rows][cols / 32] bytes, so four steps of one
// row are contiguous), into a three-slot ring: the DMA of step s carries part
// (s + 3) % 4 (rows 64 part .. 64 part + 63) of the four-step group
// (s + 3) / 4, so a group's four parts travel with the DMAs of steps
// 4 G - 3 .. 4 G and have landed before its first reader, the W reads of
// step 4 G; the slot a group refills was last read at step 4 G - 9. Needs
// cols % 512 == 0 (whole four-step groups, 16-byte aligned scale rows).
//
// Waves: p = wave & 3 takes the 64 x 128 output sub-tile (wm = p & 1 of the
// batch rows, wn = p >> 1 of the weight rows), 2 x 4 blocks of 32 x 32; wave
// group g = wave >> 2 takes the k-slice [64 g, 64 g + 64) of every step, as in
// scaled_gemm_kernel, whose fragment placement and swizzles this kernel keeps.
// Fragment reads per wave and step: 4 + 4 of 16 bytes, 2 + 4 scale words.
//
// Schedule: the ping-pong of scaled_gemm_kernel (the two wave groups half a
// step apart, a barrier after each phase) with four X stages, so that the
// X half of the fragment reads moves out of the memory phase. A wave's
// memory phase of step t issues the X DMA of step t + 3 into the stage step
// t - 1 held (and on even steps first the W pair of steps t + 2, t + 3),
// reads its W fragments and scale words of step t, waits for its
// own DMA of step t + 2 and for its LDS reads, then the barrier; its MFMA
// phase runs the step's 8 MFMAs while it reads its X fragments of step t + 1
// into a second register set. Step t + 1 is complete in LDS by then: every
// wave waited for its part of it one step earlier, before a barrier that
// both groups have passed. A stage is refilled two phases after its last
// reader's reads were waited for. Measured at 1024 x 16384 x 8192 against
// the three-stage form with every fragment read in the memory phase, three
// rounds on one box, results bit-identical: the product alone 108.1-108.3
// against 115.8-119.9 µs, the C5 graph iteration 139.7-140.6 against
// 148.2-151.0, direct 161.4-162.3 against 169.6. Reading the W half ahead
// too (212 VGPRs) gave the same product time but slower iterations: two
// waves of 212 VGPRs leave no room on a SIMD for the row kernels' waves
// beside them (2 x 56), so rmsnorm and softmax no longer run during the
// product. This form takes 198 (200 allocated), which leaves exactly that
// room.
constexpr int kWideBM = 128;
constexpr int kWideBN = 256;
constexpr int kWideXBytes = kWideBM * kBK;                  // 16 KB of X codes
constexpr int kWideXS = kWideXBytes;                        // X scale words (1 KB DMA, 512 B used)
constexpr int kWideStage = kWideXS + 1024;                  // one step's X codes and scale words
constexpr int kWideStages = 4;
constexpr int kWidePairs = kWideStages * kWideStage;        // 2 W slots: 256 rows x 128 B (two steps)
constexpr int kWidePair = kWideBN * 128;
constexpr int kWideRing = kWidePairs + 2 * kWidePair;       // W scale ring: 3 x 256 rows x 16 B
constexpr int kWideRingSlot = kWideBN * 16;
constexpr int kWideLds = kWideRing + 3 * kWideRingSlot > kExchange ? kWideRing + 3 * kWideRingSlot : kExchange;
static_assert(kWideLds <= 160 * 1024, "the wide tile's stages fit the LDS");

__global__ __launch_bounds__(kThreads, 1) void scaled_gemm_wide_kernel(float *__restrict__ out,
                                                                     const uint8_t *__restrict__ Xc,
                                                                     const uint8_t *__restrict__ Xs,
                                                                     const uint8_t *__restrict__ Wq,
                                                                     const uint8_t *__restrict__ Ws, int M,
                                                                     int N, int K) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[kWideLds];
  int tile = blockIdx.x;
  const int tiles = gridDim.x;
  if (tiles % kXcds == 0) tile = (tile % kXcds) * (tiles / kXcds) + tile / kXcds;
  const int mtiles = (M + kWideBM - 1) / kWideBM;
  const int m0 = (tile % mtiles) * kWideBM, n0 = (tile / mtiles) * kWideBN;
  const int mrows = min(kWideBM, M - m0), nrows = min(kWideBN, N - n0);
  const int Mp = padded4(M);
  const int tid = threadIdx.x, lane = tid % L2C_WAVE;
  const int wave = __builtin_amdgcn_readfirstlane(tid / L2C_WAVE);
  const int g = wave >> 2, p = wave & 3;
  const int wm = p & 1, wn = p >> 1;
  const int r = lane % 32, h = lane / 32;
  const int steps = K / kBK;
  const int groups = steps / 4;
  const int wrb = K / 2;   // E2M1 code bytes per row
  const int srb = K / 32;  // scale bytes per row
  const __amdgpu_buffer_rsrc_t rx =
      l2c::buffer_rsrc(Xc + static_cast<size_t>(m0) * K, static_cast<uint32_t>(mrows) * K);
  const __amdgpu_buffer_rsrc_t rxs = l2c::buffer_rsrc(Xs, static_cast<uint32_t>(Mp) * 4 * steps);
  const __amdgpu_buffer_rsrc_t rw =
      l2c::buffer_rsrc(Wq + static_cast<size_t>(n0) * wrb, static_cast<uint32_t>(nrows) * wrb);
  const __amdgpu_buffer_rsrc_t rws =
      l2c::buffer_rsrc(Ws + static_cast<size_t>(n0) * srb, static_cast<uint32_t>(nrows) * srb);

  // Per-lane DMA sources. X: instruction 8 k + wave (k < 2) fills rows
  // 8 (8 k + wave) + lane / 8, slot lane % 8 with chunk slot ^ xswizzle(row).
  // W pairs (128 bytes a row: step 2 p in chunks 0-3, step 2 p + 1 in 4-7):
  // instruction 8 k + wave (k < 4) fills rows 8 (8 k + wave) + lane / 8 the
  // same way. X scales (wave 4): rows 4 lane .. 4 lane + 3 (lanes past the
  // tile read the last rows again into the unused half). W scales (wave 5):
  // row 64 part + lane.
  int xsrc[2], wsrc[4];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int xrow = 8 * (8 * k + wave) + lane / 8;
    xsrc[k] = min(xrow, mrows - 1) * K + 16 * ((lane % 8) ^ xswizzle(xrow));
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int wrow = 8 * (8 * k + wave) + lane / 8;
    wsrc[k] = min(wrow, nrows - 1) * wrb + 16 * ((lane % 8) ^ xswizzle(wrow));
  }
  const int xssrc = min(16 * lane, (Mp - m0) * 4 - 16);
  const int last_pair = steps / 2 - 1;

  // The W scale part u (group u / 4, rows 64 (u % 4) + lane) into its ring
  // slot; groups past the last re-read the last group into a slot no step
  // reads any more.
  auto scale_dma = [&](int u) __attribute__((always_inline)) {
    const int part = u & 3, group = min(u >> 2, groups - 1);
    const int row = min(64 * part + lane, nrows - 1);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rws, (lds_ptr *)(lds + kWideRing + ((u >> 2) % 3) * kWideRingSlot + 64 * part * 16), 16, row * srb,
        16 * group, 0, 0);
  };
  // W pair p (steps 2 p and 2 p + 1) into slot p % 2; pairs past the last
  // re-read the last one into the slot no step reads any more.
  auto pair_dma = [&](int p) __attribute__((always_inline)) {
    unsigned char *base = lds + kWidePairs + (p & 1) * kWidePair;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr *)(base + (8 * k + wave) * 1024), 16, wsrc[k],
                                               128 * min(p, last_pair), 0, 0);
  };
  auto dma = [&](int stage, int t, int u) __attribute__((always_inline)) {
    unsigned char *base = lds + stage * kWideStage;
#pragma unroll
    for (int k = 0; k < 2; ++k)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr *)(base + (8 * k + wave) * 1024), 16, xsrc[k], kBK * t,
                                               0, 0);
    if (wave == 4)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rxs, (lds_ptr *)(base + kWideXS), 16, xssrc, Mp * 4 * t + m0 * 4, 0,
                                               0);
    if (wave == 5) scale_dma(u);
  };
  // This wave's DMA of step t + 2 has landed and its LDS reads are done; then
  // the workgroup barrier. Outstanding after the wait: the X DMA of step t + 3
  // (2 instructions, 3 on waves 4 and 5) and, on even steps, the W pair
  // issued before it (4).
  auto wait_dma_barrier = [&](bool pair_issued) __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    if (pair_issued) {
      if (wave == 4 || wave == 5)
        asm volatile("s_waitcnt vmcnt(7) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else {
      if (wave == 4 || wave == 5)
        asm volatile("s_waitcnt vmcnt(3) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto barrier = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // Fragments of lane (r, h) for the instruction over the step's blocks 2 g
  // and 2 g + 1: X rows wm * 64 + 32 i + r, chunks 4 g + h and 4 g + 2 + h; W
  // rows wn * 128 + 32 j + r, chunk 2 g + h of the step's half of the pair
  // row; scale byte 2 g + h of each row's step word (X from the stage, W from
  // the ring slot of the step's group). The swizzles of rows + 32 j equal r's.
  const int blk = 2 * g + h;
  const int xsw = xswizzle(r);
  const int xa = (wm * 64 + r) * 128;
  const int xc0 = 16 * ((4 * g + h) ^ xsw), xc1 = 16 * ((4 * g + 2 + h) ^ xsw);
  const int wr0 = wn * 128 + r;
  const int wa0 = kWidePairs + wr0 * 128 + 16 * (blk ^ xsw);        // even steps
  const int wa1 = kWidePairs + wr0 * 128 + 16 * ((4 + blk) ^ xsw);  // odd steps
  const int shift = 8 * blk;
  struct XFrag {
    u32x4 fa[2][2];
    unsigned sa[2];
  };
  XFrag fr0, fr1;
  u32x4 fb[4];
  unsigned sb[4];
  auto read_x = [&](XFrag &f, int stage) __attribute__((always_inline)) {
    const unsigned char *base = lds + stage * kWideStage;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      f.fa[i][0] = *reinterpret_cast<const u32x4 *>(base + xa + 4096 * i + xc0);
      f.fa[i][1] = *reinterpret_cast<const u32x4 *>(base + xa + 4096 * i + xc1);
      f.sa[i] = *reinterpret_cast<const unsigned *>(base + kWideXS + (wm * 64 + 32 * i + r) * 4) >> shift;
    }
  };
  auto read_w = [&](int t) __attribute__((always_inline)) {
    const unsigned char *base = lds + ((t >> 1) & 1) * kWidePair + ((t & 1) ? wa1 : wa0);
    const unsigned char *ring = lds + kWideRing + ((t >> 2) % 3) * kWideRingSlot + (t & 3) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      fb[j] = *reinterpret_cast<const u32x4 *>(base + 32 * 128 * j);
      sb[j] = *reinterpret_cast<const unsigned *>(ring + (wr0 + 32 * j) * 16) >> shift;
    }
  };
  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // Prologue: W scale parts 0-2 of group 0 (wave 5), W pair 0, then X steps
  // 0-2 with parts 3-5; the wait leaves only step 2's X outstanding, and after
  // the barrier every wave reads step 0's fragments.
  const int last = steps - 1;
  if (wave == 5) {
    scale_dma(0);
    scale_dma(1);
    scale_dma(2);
  }
  pair_dma(0);
  dma(0, 0, 3);
  dma(1, min(1, last), 4);
  dma(2, min(2, last), 5);
  wait_dma_barrier(false);
  read_x(fr0, 0);
  if (g == 1) barrier();
  // One step: the memory phase issues (on even steps) the W pair of steps
  // t + 2 and t + 3 into the slot the pair of steps t - 2 and t - 1 held and
  // the X DMA of step t + 3 into the stage step t - 1 held, reads step t's W
  // fragments and scale words, waits for this wave's DMA of step t + 2 (and so
  // for the pair of steps t + 1, t + 2 on odd steps) and for its LDS reads,
  // then the barrier; the MFMA phase runs step t's 8 MFMAs on the X fragments
  // in `use` while reading step t + 1's into `next`. A pair is issued one step
  // before its wait, as X is: the pair of steps 2 p, 2 p + 1 at step 2 p - 2,
  // waited at step 2 p - 1; its slot was last read at step 2 p - 3.
  auto step = [&](int t, bool even, XFrag &use, XFrag &next) __attribute__((always_inline)) {
    if (even) pair_dma((t >> 1) + 1);
    dma((t + 3) & 3, min(t + 3, last), t + 6);
    read_w(t);
    wait_dma_barrier(even);
    __builtin_amdgcn_s_setprio(1);
    read_x(next, (t + 1) & 3);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      i32x8 a;
#pragma unroll
      for (int c = 0; c < 4; ++c) a[c] = static_cast<int>(use.fa[i][0][c]), a[4 + c] = static_cast<int>(use.fa[i][1][c]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        i32x8 b;
#pragma unroll
        for (int c = 0; c < 4; ++c) b[c] = static_cast<int>(fb[j][c]), b[4 + c] = 0;
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc[i][j], kFmtE4M3, kFmtE2M1, 0,
                                                                    static_cast<int>(use.sa[i]), 0,
                                                                    static_cast<int>(sb[j]));
      }
    }
    // The 8 MFMAs with the 6 X reads (4 fragments, 2 scale words) between them.
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __builtin_amdgcn_s_setprio(0);
    barrier();
  };
  // steps is a multiple of 4 (cols % 512 == 0), so every pair is whole.
  for (int t = 0; t < steps; t += 2) {
    step(t, true, fr0, fr1);
    step(t + 1, false, fr1, fr0);
  }
  if (g == 0) barrier();

  // Partial sums of the two k-slices: group 1 stores, group 0 adds and writes.
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  float *exchange = reinterpret_cast<float *>(lds);
  if (g == 1) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) exchange[((p * 8 + i * 4 + j) * 16 + v) * L2C_WAVE + lane] = acc[i][j][v];
  }
  __syncthreads();
  if (g == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = wn * 128 + 32 * j + r;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int m = wm * 64 + 32 * i + 8 * (v / 4) + 4 * h + v % 4;
          const float sum = acc[i][j][v] + exchange[((p * 8 + i * 4 + j) * 16 + v) * L2C_WAVE + lane];
          if (m < mrows && n < nrows) __builtin_nontemporal_store(sum, &out[static_cast<size_t>(m0 + m) * N + n0 + n]);
        }
    }
  }
}

// Workspace views.
struct Mxfp8View {
  uint8_t *codes;
  uint8_t *scales;
};
Mxfp8View view(void *workspace, int batch, int cols) {
  uint8_t *w = static_cast<uint8_t *>(workspace);
  return {w, w + round256(static_cast<size_t>(batch) * cols)};
}

// Argument checks shared by the entry points: 0 when the shape is accepted.
int check_shape(int batch, int cols, int rows) {
  if (batch < 0 || cols <= 0 || rows < 0 || cols % kBK != 0) return hipErrorInvalidValue;
  // Per-lane byte offsets are computed in int: a tile's X rows, the W rows of
  // a tile and the whole X scale array stay below 2^31.
  if (static_cast<long long>(kBM) * cols > 0x7fffffffLL) return hipErrorInvalidValue;
  if (static_cast<long long>(padded4(batch)) * (cols / 32) > 0x7fffffffLL) return hipErrorInvalidValue;
  return hipSuccess;
}

int launch_quantizer(const Mxfp8View &v, const uint16_t *X, int batch, int cols, hipStream_t stream) {
  const int segments = (cols / 8 + 256 * kQuantChunks - 1) / (256 * kQuantChunks);
  const dim3 grid(static_cast<unsigned>(segments), static_cast<unsigned>(min(padded4(batch), 65535)));
  hipLaunchKernelGGL(quantize_mxfp8_kernel, grid, dim3(256), 0, stream, v.codes, v.scales, X, batch, padded4(batch),
                     cols);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

}  // namespace

extern "C" size_t l2c_mxfp8_workspace_bytes(int batch, int cols) {
  if (batch <= 0 || cols <= 0 || cols % kBK != 0) return 0;
  return round256(static_cast<size_t>(batch) * cols) + static_cast<size_t>(cols / kBK) * padded4(batch) * 4;
}

extern "C" int l2c_quantize_mxfp8(void *workspace, size_t workspace_bytes, const uint16_t *Xbf16, int batch,
                                  int cols, hipStream_t stream) {
  if (const int e = check_shape(batch, cols, 0)) return e;
  if (batch == 0) return hipSuccess;
  if (!workspace || !Xbf16 || !l2c_aligned16(Xbf16) || !l2c_aligned16(workspace)) return hipErrorInvalidValue;
  if (workspace_bytes < l2c_mxfp8_workspace_bytes(batch, cols)) return hipErrorInvalidValue;
  return launch_quantizer(view(workspace, batch, cols), Xbf16, batch, cols, stream);
}

extern "C" int l2c_matmul_qs(float *out, const void *Xbf16, const void *Wq, const void *scales, int fmt, int batch,
                             int cols, int rows, void *workspace, size_t workspace_bytes, hipStream_t stream) {
  if (fmt != L2C_Q_MXFP4 && fmt != L2C_Q_FP8) return hipErrorInvalidValue;
  if (const int e = check_shape(batch, cols, rows)) return e;
  if (batch == 0 || rows == 0) return hipSuccess;
  if (!out || !Xbf16 || !Wq || !scales || !workspace) return hipErrorInvalidValue;
  if (!l2c_aligned16(Xbf16) || !l2c_aligned16(Wq) || !l2c_aligned16(workspace) ||
      (reinterpret_cast<uintptr_t>(scales) & 3u))
    return hipErrorInvalidValue;
  if (workspace_bytes < l2c_mxfp8_workspace_bytes(batch, cols)) return hipErrorInvalidValue;
  if (static_cast<long long>(kBN) * (fmt == L2C_Q_MXFP4 ? cols / 2 : cols) > 0x7fffffffLL) return hipErrorInvalidValue;
  const long long tiles = static_cast<long long>((batch + kBM - 1) / kBM) * ((rows + kBN - 1) / kBN);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  const Mxfp8View v = view(workspace, batch, cols);
  if (const int e = launch_quantizer(v, static_cast<const uint16_t *>(Xbf16), batch, cols, stream)) return e;
  const uint8_t *W = static_cast<const uint8_t *>(Wq);
  // Wide tiles for MXFP4 weights in whole four-step scale groups whose 16-byte
  // scale rows are aligned; the 256 x 128 tile otherwise.
  const long long wide_tiles =
      static_cast<long long>((batch + kWideBM - 1) / kWideBM) * ((rows + kWideBN - 1) / kWideBN);
  if (fmt == L2C_Q_MXFP4 && cols % 512 == 0 && l2c_aligned16(scales) &&
      static_cast<long long>(kWideBN) * (cols / 2) <= 0x7fffffffLL && wide_tiles <= 0x7fffffffLL) {
    hipLaunchKernelGGL(scaled_gemm_wide_kernel, dim3(static_cast<unsigned>(wide_tiles)), dim3(kThreads), 0, stream,
                       out, v.codes, v.scales, W, static_cast<const uint8_t *>(scales), batch, rows, cols);
  } else if (fmt == L2C_Q_MXFP4)
    hipLaunchKernelGGL(scaled_gemm_kernel<L2C_Q_MXFP4>, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, stream,
                       out, v.codes, v.scales, W, scales, batch, rows, cols);
  else
    hipLaunchKernelGGL(scaled_gemm_kernel<L2C_Q_FP8>, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, stream,
                       out, v.codes, v.scales, W, scales, batch, rows, cols);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

namespace {

// Device address of `scratch` on each device, resolved once per device with
// that device current.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void *g_scratch[kMaxDevices] = {};

int scratch_on_current_device(void **ptr) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return e;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> hold(g_scratch_lock);
  if (!g_scratch[device]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch[device] = p;
  }
  *ptr = g_scratch[device];
  return hipSuccess;
}

}  // namespace

extern "C" int l2c_matmul_qs_static(float *out, const void *Xbf16, const void *Wq, const void *scales, int fmt,
                                    int batch, int cols, int rows, hipStream_t stream) {
  if (const int e = check_shape(batch, cols, rows)) return e;
  if (batch == 0 || rows == 0) return l2c_matmul_qs(out, Xbf16, Wq, scales, fmt, batch, cols, rows, nullptr, 0, stream);
  const size_t need = l2c_mxfp8_workspace_bytes(batch, cols);
  if (need == 0 || need > static_cast<size_t>(L2C_QS_STATIC_SCRATCH_BYTES)) return hipErrorInvalidValue;
  void *ws = nullptr;
  if (const int e = scratch_on_current_device(&ws)) return e;
  return l2c_matmul_qs(out, Xbf16, Wq, scales, fmt, batch, cols, rows, ws, L2C_QS_STATIC_SCRATCH_BYTES, stream);
}

int l2c_scgemm_occupancy(int fmt, bool wide, int *blocks_per_cu) {
  const void *fn = wide ? reinterpret_cast<const void *>(scaled_gemm_wide_kernel)
                   : fmt == L2C_Q_MXFP4 ? reinterpret_cast<const void *>(scaled_gemm_kernel<L2C_Q_MXFP4>)
                                        : reinterpret_cast<const void *>(scaled_gemm_kernel<L2C_Q_FP8>);
  return static_cast<int>(hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, fn, kThreads, 0));
}
