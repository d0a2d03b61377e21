// Quantized-weight contraction out[b][r] = sum_k X[b][k] * deq(W)[r][k] with
// bf16 activations and MXFP4, per-row-scaled fp8 e4m3 or bf16 weights, plus
// the device quantizers that produce those weights. The bf16-weight form is
// the classifier of the lowprec bf16 and NVFP4 cases (an optional device
// alpha multiplies each output).
//
// Kernel design (gfx950):
//  * The activations are bf16 and must stay bf16 (the oracle multiplies the
//    exact bf16 values), so the product runs on the bf16 matrix cores
//    (v_mfma_f32_32x32x16_bf16, fp32 accumulation).
//  * Weights are converted exactly to bf16 in registers by the gfx950 scaled
//    conversions (v_cvt_scalef32_pk_bf16_fp4 / _fp8: two codes to two bf16,
//    times the block scale 2^(s - 127)): an e2m1 magnitude times a power of
//    two, or an e4m3 value, has at most 4 significant bits, so the bf16 value
//    is exact. The fp8 row scale is applied once per output in the epilogue.
//  * Tile 256 (batch) x 128 (rows) x 64 (k), 8 wavefronts of 64 x 64 (2 x 2
//    blocks of 32 x 32); 4 x 64 = 256 tiles at 1024 x 8192, one per CU.
//  * Each k-step's X slab (256 rows x 128 B), W codes (128 rows x 32 or 64 B)
//    and MXFP4 block scales (converted once to fp32 by the staging thread)
//    pass through a three-stage LDS ring: step t multiplies stage t % 3,
//    stores step t + 2 into stage (t + 2) % 3, and reads step t + 1's
//    fragments into registers before the step's barrier, so no wave waits on
//    LDS latency after a barrier. Global loads run four steps ahead through
//    two register sets. Every thread stages the same amount (branch-free).
//  * Buffer loads: per-lane byte offsets are computed once (rows past the
//    operand clamped) and the k-step is a scalar offset. A partial last step
//    (K % 64 == 32) runs after the loop; its lanes past K read in-bounds
//    codes and get zero B operands.
//  * LDS layouts are bank-conflict free for both the staging stores and the
//    fragment reads: X rows are padded to 144 B; W rows are unpadded with
//    their 16-byte chunks XOR-swizzled by row bits; scales are a separate
//    [128][2] fp32 array.
//  * k permutation: within a step, lane (r, h) (r = lane % 32, h = lane / 32)
//    of MFMA q in 0..3 supplies k = 32h + 8q + j (j < 8) for both operands, so
//    a lane's W codes for the step are 32 consecutive k (16 contiguous bytes of
//    MXFP4) and its X fragment of MFMA q is 8 contiguous bf16 in LDS. MFMA
//    operand layout: lane l supplies A[l % 32][8 * (l / 32) + 0..7] and
//    B[8 * (l / 32) + 0..7][l % 32]; the accumulator layout matches the fp32
//    kernel's.
//  * Workgroup order is remapped per XCD as in the fp32 kernel.
//
// Encodings (bit-identical to the host encoders of the harness):
//  * e2m1: magnitudes {0, .5, 1, 1.5, 2, 3, 4, 6}, bit 3 the sign; nearest,
//    ties to the even code, saturating at 6, -0 -> +0. Two codes per byte,
//    even k in the low nibble. Block of 32 k: e8m0 scale 2^(s - 127) with
//    s - 127 = floor(log2(amax / 6)) clamped to [-127, 127].
//  * e4m3 (OCP, bias 7, max 448, no infinities): nearest-even, saturating.
#include <type_traits>

#include "l2c_common.h"
#include "l2c_formats.h"
#include "../../include/l2c.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 256;
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kWavesM = 4;
constexpr int kWavesN = 2;
constexpr int kThreads = kWavesM * kWavesN * L2C_WAVE;  // 512
constexpr int kFragM = kBM / kWavesM / 32;              // 2
constexpr int kFragN = kBN / kWavesN / 32;              // 2
constexpr int kStages = 3;
constexpr int kXStride = 144;                           // LDS bytes per X row (64 bf16 + 16 pad)
constexpr int kXChunks = kBM * (kBK / 8) / kThreads;    // 16-byte X chunks per thread and step: 4
constexpr int kXcds = 8;
// The X tile of one workgroup must stay addressable with the per-lane byte
// offsets, row * K * 2 computed in (signed) int.
constexpr long long kMaxTileBytes = 0x7fffffffLL;

// Per-format staging geometry. W rows hold the step's codes (32 bytes of
// MXFP4 or 64 of fp8) with 16-byte chunks XOR-swizzled by row bits; MXFP4
// block scales follow as fp32 [kBN][2].
constexpr int kFmtBf16 = 2;  // bf16 weights (l2c_matmul_bf16)

template <int FMT>
struct Geometry {
  // Code bytes per W row and step: 64 k of MXFP4, fp8 or bf16.
  static constexpr int kWRow = FMT == L2C_Q_MXFP4 ? 32 : FMT == L2C_Q_FP8 ? 64 : 128;
  static constexpr int kWBytes = kWRow * kBN / kThreads;      // code bytes staged per thread
  static constexpr int kWReads = kWRow / 32;                  // 16-byte code reads per block
  static constexpr int kXStage = kBM * kXStride;
  static constexpr int kSStage = kXStage + kBN * kWRow;
  static constexpr int kStage = kSStage + (FMT == L2C_Q_MXFP4 ? kBN * 8 : 0);
  // Chunk swizzle: 16 lanes reading chunk c of 16 consecutive rows (or 32
  // lanes storing 8 rows) touch 64 distinct banks.
  static __device__ __forceinline__ int swizzle(int row) {
    return FMT == L2C_Q_MXFP4 ? (row >> 3) & 1 : FMT == L2C_Q_FP8 ? (row >> 2) & 3 : (row >> 1) & 7;
  }
};

// ---------------------------------------------------------------------------
// Element encoders / decoders.

using l2c::e2m1_code;
using l2c::e4m3_code;

__device__ __forceinline__ int mxfp4_exponent(float amax) {
  const unsigned bits = __float_as_uint(amax);
  const int be = static_cast<int>((bits >> 23) & 0xffu);
  if (be == 0) return -127;  // zero or subnormal: the clamp decides
  const int x = be - 127 - 3 + static_cast<int>((bits >> 22) & 1u);
  return min(127, max(-127, x));
}

__device__ __forceinline__ float pow2f(int e) {  // e in [-126, 127]
  return __uint_as_float(static_cast<unsigned>(e + 127) << 23);
}

// ---------------------------------------------------------------------------
// Quantizers (setup work).

// One thread per 32-element block of a row.
__global__ void quantize_mxfp4_kernel(uint8_t *codes, uint8_t *scales, const float *W,
                                      long long blocks) {
  const long long blk = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (blk >= blocks) return;
  const float *w = W + blk * 32;
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(w[i]));
  const int x = mxfp4_exponent(amax);
  const float inv = pow2f(-x);  // -x in [-127, 127]; 2^-127 never needed (x <= 125)
  uint32_t packed[4] = {0, 0, 0, 0};
  if (amax > 0.0f) {
    for (int i = 0; i < 32; ++i)
      packed[i / 8] |= e2m1_code(w[i] * inv) << (4 * (i % 8));
  }
  uint32_t *out = reinterpret_cast<uint32_t *>(codes + blk * 16);
  for (int i = 0; i < 4; ++i) out[i] = packed[i];
  scales[blk] = static_cast<uint8_t>(x + 127);
}

// One block per row.
__global__ __launch_bounds__(256) void quantize_fp8_kernel(uint8_t *codes, float *scales,
                                                           const float *W, int cols) {
  __shared__ float slots[8];
  const size_t off = static_cast<size_t>(blockIdx.x) * cols;
  float amax = 0.0f;
  for (int k = threadIdx.x; k < cols; k += blockDim.x) amax = fmaxf(amax, fabsf(W[off + k]));
  amax = l2c::block_max(amax, slots);
  const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
  for (int k = threadIdx.x; k < cols; k += blockDim.x)
    codes[off + k] = static_cast<uint8_t>(e4m3_code(W[off + k] / scale));
  if (threadIdx.x == 0) scales[blockIdx.x] = scale;
}

__global__ void to_bf16_kernel(uint16_t *out, const float *in, size_t n) {
  const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const unsigned bits = __float_as_uint(in[i]);
  if ((bits & 0x7f800000u) == 0x7f800000u) {
    out[i] = static_cast<uint16_t>(bits >> 16);
    return;
  }
  // Nearest even of the two finite neighbours: a finite value never becomes
  // infinite (experiments/blackwell/lowprec/reference.cpp:84-96 picks between
  // the truncation and the next finite magnitude).
  unsigned r = (bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16;
  if ((r & 0x7fffu) == 0x7f80u) --r;
  out[i] = static_cast<uint16_t>(r);
}

// ---------------------------------------------------------------------------
// The contraction.

template <int FMT>
__global__ __launch_bounds__(kThreads) void qgemm_kernel(float *__restrict__ out,
                                                         const uint16_t *__restrict__ X,
                                                         const uint8_t *__restrict__ Wq,
                                                         const void *__restrict__ scales,
                                                         int M, int N, int K) {
  using G = Geometry<FMT>;
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  __shared__ __attribute__((aligned(16))) unsigned char lds[kStages * G::kStage];

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

  const int wrow_bytes = FMT == L2C_Q_MXFP4 ? K / 2 : FMT == L2C_Q_FP8 ? K : 2 * K;
  const __amdgpu_buffer_rsrc_t rx =
      l2c::buffer_rsrc(X + static_cast<size_t>(m0) * K, static_cast<uint32_t>(mrows) * K * 2u);
  const __amdgpu_buffer_rsrc_t rw =
      l2c::buffer_rsrc(Wq + static_cast<size_t>(n0) * wrow_bytes, static_cast<uint32_t>(nrows) * wrow_bytes);
  const __amdgpu_buffer_rsrc_t rs = l2c::buffer_rsrc(
      static_cast<const uint8_t *>(scales) + (FMT == L2C_Q_MXFP4 ? static_cast<size_t>(n0) * (K / 32) : 0),
      FMT == L2C_Q_MXFP4 ? static_cast<uint32_t>(nrows) * (K / 32) : 4u);

  // Staging assignments (global byte offsets without the step part, LDS
  // offsets within a stage).
  int xg[kXChunks], xs[kXChunks];
#pragma unroll
  for (int v = 0; v < kXChunks; ++v) {
    const int id = v * kThreads + tid, row = id / 8, c = id % 8;
    xg[v] = min(row, mrows - 1) * K * 2 + 16 * c;
    xs[v] = row * kXStride + 16 * c;
  }
  const int wrow = tid / (G::kWRow / G::kWBytes);
  const int wbyte = G::kWBytes * (tid % (G::kWRow / G::kWBytes));
  const int wg = min(wrow, nrows - 1) * wrow_bytes + wbyte;
  const int ws = G::kXStage + wrow * G::kWRow + (((wbyte >> 4) ^ G::swizzle(wrow)) << 4) + (wbyte & 15);
  // bf16: the thread's second 16-byte chunk.
  const int ws1 = G::kXStage + wrow * G::kWRow + ((((wbyte >> 4) + 1) ^ G::swizzle(wrow)) << 4);
  // MXFP4 scales: threads t and t + 256 stage the same (row, half) word.
  const int srow = (tid & 255) / 2, shalf = tid & 1;
  const int sg = min(srow, nrows - 1) * (K / 32) + shalf;
  const int ss = G::kSStage + (srow * 2 + shalf) * 4;

  u32x4 gx[2][kXChunks];
  u32x4 gw4[2];
  u32x4 gw8[2];
  u32x2 gw2[2];
  uint32_t gs[2];
  auto gload = [&](auto set, int t) __attribute__((always_inline)) {
    constexpr int st = decltype(set)::value;
#pragma unroll
    for (int v = 0; v < kXChunks; ++v) gx[st][v] = __builtin_amdgcn_raw_buffer_load_b128(rx, xg[v], 128 * t, 0);
    if constexpr (G::kWBytes >= 16) gw4[st] = __builtin_amdgcn_raw_buffer_load_b128(rw, wg, G::kWRow * t, 0);
    else gw2[st] = __builtin_amdgcn_raw_buffer_load_b64(rw, wg, G::kWRow * t, 0);
    if constexpr (G::kWBytes == 32) gw8[st] = __builtin_amdgcn_raw_buffer_load_b128(rw, wg + 16, G::kWRow * t, 0);
    if constexpr (FMT == L2C_Q_MXFP4) gs[st] = __builtin_amdgcn_raw_buffer_load_b8(rs, sg, 2 * t, 0);
  };
  auto lstore = [&](auto set, int stage) __attribute__((always_inline)) {
    constexpr int st = decltype(set)::value;
    unsigned char *base = lds + stage * G::kStage;
#pragma unroll
    for (int v = 0; v < kXChunks; ++v) *reinterpret_cast<u32x4 *>(base + xs[v]) = gx[st][v];
    if constexpr (G::kWBytes >= 16) *reinterpret_cast<u32x4 *>(base + ws) = gw4[st];
    else *reinterpret_cast<u32x2 *>(base + ws) = gw2[st];
    if constexpr (G::kWBytes == 32) *reinterpret_cast<u32x4 *>(base + ws1) = gw8[st];
    if constexpr (FMT == L2C_Q_MXFP4) {
      // Block scale 2^(s - 127) as fp32 (s = 0 is the subnormal 2^-127).
      const uint32_t e = gs[st] & 0xffu;
      *reinterpret_cast<uint32_t *>(base + ss) = e == 0 ? 0x00400000u : (e << 23);
    }
  };

  f32x16 acc[kFragM][kFragN];
#pragma unroll
  for (int i = 0; i < kFragM; ++i)
#pragma unroll
    for (int j = 0; j < kFragN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // This lane's fragments: X row wm * 64 + 32 i + r, W row brow + 32 j.
  const int a_off = (wm * kFragM * 32 + r) * kXStride + 64 * h;
  const int brow = wn * kFragN * 32 + r;
  const int s_off = G::kSStage + (brow * 2 + h) * 4;
  struct Frags {
    u32x4 w[kFragN][G::kWReads];
    uint32_t s[kFragN];
    u32x4 a[kFragM][4];
  };
  auto read_frags = [&](int stage, Frags &f) __attribute__((always_inline)) {
    const unsigned char *base = lds + stage * G::kStage;
#pragma unroll
    for (int j = 0; j < kFragN; ++j) {
#pragma unroll
      for (int v = 0; v < G::kWReads; ++v) {
        const int row = brow + 32 * j;
        const int chunk = (G::kWReads * h + v) ^ G::swizzle(row);
        f.w[j][v] = *reinterpret_cast<const u32x4 *>(base + G::kXStage + row * G::kWRow + 16 * chunk);
      }
      if constexpr (FMT == L2C_Q_MXFP4)
        f.s[j] = *reinterpret_cast<const uint32_t *>(base + s_off + j * 32 * 8);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < kFragM; ++i)
        f.a[i][q] = *reinterpret_cast<const u32x4 *>(base + a_off + i * 32 * kXStride + 16 * q);
  };
  // B operand of MFMA q for block j: W[k = 32h + 8q + 0..7] of row brow + 32 j;
  // zero when kok is false (lanes past K in the partial last step).
  auto mma = [&](const Frags &f, bool kok) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      bf16x8 b[kFragN];
#pragma unroll
      for (int j = 0; j < kFragN; ++j) {
        uint32_t d[4];
        if constexpr (FMT == L2C_Q_MXFP4) {
          // Lanes past K get zero codes, not a zero scale: the scaled
          // conversion reads only the scale's exponent field, so a scale of
          // 0.0 multiplies by 2^-127 rather than by zero.
          const float scale = __uint_as_float(f.s[j]);
          const uint32_t c = kok ? f.w[j][0][q] : 0u;  // codes k = 8q .. 8q + 7, two per byte
          d[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, scale, 0));
          d[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, scale, 1));
          d[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, scale, 2));
          d[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, scale, 3));
        } else if constexpr (FMT == kFmtBf16) {
          d[0] = kok ? f.w[j][q][0] : 0u;
          d[1] = kok ? f.w[j][q][1] : 0u;
          d[2] = kok ? f.w[j][q][2] : 0u;
          d[3] = kok ? f.w[j][q][3] : 0u;
        } else {
          const uint32_t c0 = kok ? f.w[j][q / 2][2 * (q % 2)] : 0u;
          const uint32_t c1 = kok ? f.w[j][q / 2][2 * (q % 2) + 1] : 0u;
          d[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c0, 1.0f, false));
          d[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c0, 1.0f, true));
          d[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c1, 1.0f, false));
          d[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c1, 1.0f, true));
        }
        b[j] = __builtin_bit_cast(bf16x8, make_uint4(d[0], d[1], d[2], d[3]));
      }
#pragma unroll
      for (int i = 0; i < kFragM; ++i)
#pragma unroll
        for (int j = 0; j < kFragN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, f.a[i][q]), b[j],
                                                              acc[i][j], 0, 0, 0);
    }
  };

  Frags fr[2];
  const int nfull = K / kBK;
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  if (nfull > 0) {
    // Steps past the last are clamped to it: redundant in-bounds loads whose
    // copies are never read.
    const int last = nfull - 1;
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
      mma(fr[st], true);
      lstore(set, wr);
      gload(set, min(t + 4, last));
      __syncthreads();
      rd = nx;
      ++t;
    };
    for (; t + 2 <= nfull;) {
      step(I0());
      step(I1());
    }
    if (t < nfull) mma(fr[0], true);
  }
  if (K % kBK != 0) {
    // Half step at k0 = 64 * nfull: chunks past K read in-bounds data from
    // the valid half, and the B operands of lanes h = 1 are zero.
    __syncthreads();
    const int t2 = nfull;
#pragma unroll
    for (int v = 0; v < kXChunks; ++v) {
      const int c = (v * kThreads + tid) % 8;
      gx[0][v] = __builtin_amdgcn_raw_buffer_load_b128(rx, xg[v] - (c >= 4 ? 64 : 0), 128 * t2, 0);
    }
    const int half = G::kWRow / 2;
    const int wgo = wg - (wbyte >= half ? half : 0);
    if constexpr (G::kWBytes >= 16) gw4[0] = __builtin_amdgcn_raw_buffer_load_b128(rw, wgo, G::kWRow * t2, 0);
    else gw2[0] = __builtin_amdgcn_raw_buffer_load_b64(rw, wgo, G::kWRow * t2, 0);
    if constexpr (G::kWBytes == 32) gw8[0] = __builtin_amdgcn_raw_buffer_load_b128(rw, wgo + 16, G::kWRow * t2, 0);
    if constexpr (FMT == L2C_Q_MXFP4) gs[0] = __builtin_amdgcn_raw_buffer_load_b8(rs, sg - shalf, 2 * t2, 0);
    lstore(I0(), 0);
    __syncthreads();
    read_frags(0, fr[0]);
    mma(fr[0], h == 0);
  }

#pragma unroll
  for (int j = 0; j < kFragN; ++j) {
    const int n = brow + 32 * j;
    float rs_ = 1.0f;
    if constexpr (FMT == L2C_Q_FP8) rs_ = n < nrows ? static_cast<const float *>(scales)[n0 + n] : 0.0f;
    if constexpr (FMT == kFmtBf16) rs_ = scales ? *static_cast<const float *>(scales) : 1.0f;  // alpha
#pragma unroll
    for (int i = 0; i < kFragM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = wm * kFragM * 32 + 32 * i + 8 * (v / 4) + 4 * h + v % 4;
        if (m < mrows && n < nrows) out[static_cast<size_t>(m0 + m) * N + n0 + n] = acc[i][j][v] * rs_;
      }
    }
  }
}

}  // namespace

int l2c_qgemm_launch_shape(int fmt, int batch, int cols, int rows, int *grid, int *block,
                           int *blocks_per_cu) {
  if (fmt != L2C_Q_MXFP4 && fmt != L2C_Q_FP8) return hipErrorInvalidValue;
  *grid = ((batch + kBM - 1) / kBM) * ((rows + kBN - 1) / kBN);
  *block = kThreads;
  if (cols % 64 == 0) {
    *grid = static_cast<int>(l2c_qgemm_ks_tiles(fmt, batch, rows));
    return l2c_qgemm_ks_occupancy(fmt, blocks_per_cu);
  }
  const void *fn = fmt == L2C_Q_MXFP4 ? reinterpret_cast<const void *>(qgemm_kernel<L2C_Q_MXFP4>)
                                      : reinterpret_cast<const void *>(qgemm_kernel<L2C_Q_FP8>);
  return static_cast<int>(hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, fn, kThreads, 0));
}

extern "C" int l2c_matmul_q(float *out, const void *Xbf16, const void *Wq, const void *scales,
                            int fmt, int batch, int cols, int rows, hipStream_t stream) {
  if (batch < 0 || cols <= 0 || rows < 0 || cols % 32 != 0) return hipErrorInvalidValue;
  if (fmt != L2C_Q_MXFP4 && fmt != L2C_Q_FP8) return hipErrorInvalidValue;
  if (batch == 0 || rows == 0) return hipSuccess;
  if (!out || !Xbf16 || !Wq || !scales) return hipErrorInvalidValue;
  if (!l2c_aligned16(Xbf16) || !l2c_aligned16(Wq)) return hipErrorInvalidValue;
  if (static_cast<long long>(kBM) * cols * 2 > kMaxTileBytes) return hipErrorInvalidValue;
  const long long tiles =
      static_cast<long long>((batch + kBM - 1) / kBM) * ((rows + kBN - 1) / kBN);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(tiles)), block(kThreads);
  const uint16_t *X = static_cast<const uint16_t *>(Xbf16);
  const uint8_t *W = static_cast<const uint8_t *>(Wq);
  if (cols % 64 == 0 && (fmt == L2C_Q_FP8 || (reinterpret_cast<uintptr_t>(scales) & 1u) == 0))
    return l2c_matmul_q_ks(out, X, W, scales, fmt, batch, cols, rows, stream);
  if (fmt == L2C_Q_MXFP4)
    hipLaunchKernelGGL(qgemm_kernel<L2C_Q_MXFP4>, grid, block, 0, stream, out, X, W, scales, batch,
                       rows, cols);
  else
    hipLaunchKernelGGL(qgemm_kernel<L2C_Q_FP8>, grid, block, 0, stream, out, X, W, scales, batch,
                       rows, cols);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

extern "C" int l2c_quantize_mxfp4(uint8_t *codes, uint8_t *scales, const float *W, int rows,
                                  int cols, hipStream_t stream) {
  if (rows < 0 || cols <= 0 || cols % 32 != 0) return hipErrorInvalidValue;
  if (rows == 0) return hipSuccess;
  if (!codes || !scales || !W || !l2c_aligned16(codes)) return hipErrorInvalidValue;
  const long long blocks = static_cast<long long>(rows) * (cols / 32);
  const long long grid = (blocks + 255) / 256;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(quantize_mxfp4_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                     stream, codes, scales, W, blocks);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

extern "C" int l2c_quantize_fp8(uint8_t *codes, float *scales, const float *W, int rows, int cols,
                                hipStream_t stream) {
  if (rows < 0 || cols <= 0) return hipErrorInvalidValue;
  if (rows == 0) return hipSuccess;
  if (!codes || !scales || !W) return hipErrorInvalidValue;
  hipLaunchKernelGGL(quantize_fp8_kernel, dim3(rows), dim3(256), 0, stream, codes, scales, W, cols);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

extern "C" int l2c_to_bf16(uint16_t *out, const float *in, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  if (!out || !in) return hipErrorInvalidValue;
  const size_t grid = (n + 255) / 256;
  if (grid > 0x7fffffffULL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(to_bf16_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, stream, out,
                     in, n);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

// bf16 weights through this kernel: l2c_matmul_bf16 (l2c_bfgemm.hip) uses it for
// K % 64 == 32, which its own kernel does not take.
int l2c_matmul_bf16_split(float *out, const uint16_t *X, const uint16_t *W, const float *alpha, int batch, int cols,
                          int rows, hipStream_t stream) {
  if (batch < 0 || cols <= 0 || rows < 0 || cols % 32 != 0) return hipErrorInvalidValue;
  if (batch == 0 || rows == 0) return hipSuccess;
  if (!out || !X || !W || !l2c_aligned16(X) || !l2c_aligned16(W)) return hipErrorInvalidValue;
  if (static_cast<long long>(kBM) * cols * 2 > kMaxTileBytes) return hipErrorInvalidValue;
  const long long tiles =
      static_cast<long long>((batch + kBM - 1) / kBM) * ((rows + kBN - 1) / kBN);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(qgemm_kernel<kFmtBf16>, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, stream, out,
                     X, reinterpret_cast<const uint8_t *>(W), static_cast<const void *>(alpha), batch, rows, cols);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}
