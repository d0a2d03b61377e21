// Quantized-weight contraction out[b][r] = sum_k X[b][k] * deq(W)[r][k] for
// K % 64 == 0: bf16 activations, MXFP4 (E2M1 codes, one E8M0 scale per 32 k)
// or per-row-scaled fp8 E4M3 weights, in the layouts l2c_quantize_mxfp4 and
// l2c_quantize_fp8 write (codes row-major, MXFP4 scales [rows][K/32]).
// l2c_matmul_q routes K % 64 == 32 to the kernel in l2c_qgemm.hip.
//
// Kernel design:
//  * The product runs on the bf16 matrix cores (v_mfma_f32_32x32x16_bf16);
//    the weight codes are converted exactly to bf16 in registers by the
//    gfx950 scaled conversions (v_cvt_scalef32_pk_bf16_fp4 / _fp8), an E2M1
//    value times 2^(s - 127) or an E4M3 value having at most 4 significant
//    bits. The conversion reads only the exponent field of its fp32 scale, so
//    the E8M0 byte shifted into that field is the scale for every byte value
//    (byte 0, 0.0f, scales by 2^-127). The fp8 row scale multiplies each
//    output in the epilogue.
//  * Tile 256 (batch) x 128 (rows) x 64 (k per step) for MXFP4, 128 x 256 x 64
//    for fp8, 8 wavefronts in k-slice pairs: waves w and w + 4 share a SIMD
//    and a 128 x 64 output sub-tile (2 x 2 or 1 x 4 of them per group) and
//    take the step's k-chunks 2g, 2g + 1 (g = w / 4); lane (r, h) of MFMA q
//    supplies k = 32h + 8q + 0..7 for both operands, so a lane's codes for its
//    two chunks are 8 contiguous bytes (MXFP4, one scale block h) or 16 (fp8).
//    The pairs' partial sums are added once at the end through LDS.
//  * Ping-pong schedule: the two waves of a SIMD run half a step apart. Group 0
//    (waves 0-3) runs its memory phase of step t -- the fragment reads of step t,
//    the DMA of step t + 3 into the stage step t - 1 held, the conversions of
//    step t, a wait for its DMA of step t + 1 -- while group 1 (waves 4-7) runs
//    its 16 MFMAs of step t - 1 at raised wave priority; then the roles swap. A
//    workgroup barrier ends each phase, so each SIMD's matrix core takes one
//    wave's MFMAs while the other wave waits on LDS and memory. Group 1 takes one
//    extra barrier at the start and group 0 one at the end, so every wave passes
//    the same number of barriers.
//  * LDS DMA staging (buffer_load ... lds): X 32 KB (MXFP4) or 16 KB (fp8) a
//    step in 1-KB instructions of 8 rows; W codes 4 KB (MXFP4, waves 0-3) or
//    16 KB (fp8, two a wave); MXFP4 scales as 2-byte DMAs, one row a lane
//    (waves 4, 5), each landing zero-extended in its own LDS word (a 2-byte
//    DMA writes lane i's bytes at word i). Four stages (146 KB MXFP4, 128 KB
//    fp8): a stage is free once both groups have read it, and a step's DMA
//    has three steps to land.
//  * 16-byte chunks of LDS rows are XOR-swizzled by row bits (X: bits 1..3;
//    W: bit 3 for 32-byte MXFP4 rows, bits 2..3 for 64-byte fp8 rows), applied
//    on the DMA's source side, so the fragment reads avoid bank conflicts
//    (MXFP4's 8-byte reads keep a two-way conflict on 2 KB a wave and step).
//  * Measured at 1024 x 16384 x 8192 against the earlier schedule (both
//    waves of a SIMD in step, one barrier a step; the matrix cores busy 55% of
//    the time): MXFP4 214 against 226-229 µs, fp8 206 against 223-228 µs.
//    Timing probes with work removed: without the DMA 164 / 175 µs, without
//    the DMA and the fragment reads 149 / 162 µs (the MFMAs alone on these
//    operands); removing the conversions or the DMA wait changes nothing.
//    fp8 on the 256 x 128 tile took four 40 KB stages, the CU's whole LDS,
//    so in the C5 iteration the row kernels could not run beside it (three
//    stages there, one step for the DMA, measured 213 µs). The 128 x 256
//    tile gives the same results bit for bit with 32 KB stages: alone within
//    1% (209 against 207 µs on the harness's weights), the graph iteration
//    252 against 281 µs. MXFP4 on it measured 226 against 216 µs (213 against
//    197.5 µs with the present schedule, three rounds on one box, bit-identical)
//    and keeps 256 x 128. Issuing the fragment reads ahead of the DMA measured 1-1.3%
//    faster than the DMA first (fp8 201.4-202.9 against 203.3-204.7 µs,
//    MXFP4 203.0-203.5 against 205.6-206.0 µs).
//  * Every access is in bounds by construction: rows past the operand are
//    clamped per lane to its last row; those rows are never stored.
#include "l2c_common.h"
#include "../../include/l2c.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_ptr;

constexpr int kThreads = 512;
constexpr int kXcds = 8;
constexpr int kExchange = 131072;  // 4 sub-tiles x 8 blocks x 16 values x 64 lanes x 4 B

// A tile is BM batch rows x 32768 / BM weight rows (256 x 128 or 128 x 256); a
// wave's sub-tile is always 128 x 64, so a wave group holds BM / 128 x BN / 64
// of them.
template <int FMT, int STAGES, int BM>
struct Layout {
  static constexpr int kStages = STAGES;
  static constexpr bool kMx = FMT == L2C_Q_MXFP4;
  static constexpr int kBM = BM;
  static constexpr int kBN = 32768 / BM;
  static constexpr int kWavesM = BM / 128;        // sub-tiles along the batch
  static constexpr int kXBytes = BM * 128;        // BM rows x 64 bf16
  static constexpr int kXDma = BM / 64;           // X DMAs a wave issues a step (8 rows x 128 B each)
  static constexpr int kWRow = kMx ? 32 : 64;     // code bytes per W row and step
  static constexpr int kLanesPerRow = kWRow / 16;
  static constexpr int kWRowsPerDma = 64 / kLanesPerRow;
  static constexpr int kWDma = kBN / kWRowsPerDma;  // W DMAs a step, instruction q on wave q % 8
  static constexpr int kSDma = kMx ? kBN / 64 : 0;  // MXFP4 scale DMAs a step, on waves 4, 5, ...
  static constexpr int kSOff = kXBytes + kBN * kWRow;
  static constexpr int kStage = kSOff + (kMx ? kBN * 4 : 0);
  static constexpr int kLds = kStages * kStage > kExchange ? kStages * kStage : kExchange;
  // The wait for a step's DMA lets STAGES - 2 newer steps stay in flight,
  // counted at the fewest DMAs any wave issues a step (4 for the 256-row
  // tile, whose waves issue 4 or 5; 4 for fp8 and 3 for MXFP4 on the 128-row
  // tile): exact for those waves, stricter for the others.
  static constexpr int kWait = (BM == 256 ? 4 : kXDma + kWDma / 8) * (STAGES - 2);
  static __device__ __forceinline__ int wswizzle(int row) { return kMx ? (row >> 3) & 1 : (row >> 2) & 3; }
};

__device__ __forceinline__ int xswizzle(int row) { return (row >> 1) & 7; }

// One step's DMA by one wave into the stage at `base` (the per-lane sources
// are described at the kernel). The W step stride comes in as `wstep`, a
// plain argument.
template <int FMT, int STAGES, int BM>
__device__ __forceinline__ void issue_step_dma(unsigned char *base, int t, int wave, __amdgpu_buffer_rsrc_t rx,
                                               __amdgpu_buffer_rsrc_t rw, __amdgpu_buffer_rsrc_t rs,
                                               const int (&xsrc)[4], const int (&wsrc)[2], int ssrc, int wstep) {
  using L = Layout<FMT, STAGES, BM>;
#pragma unroll
  for (int k = 0; k < (L::kWDma + 7) / 8; ++k)
    if (8 * k + wave < L::kWDma)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr *)(base + L::kXBytes + (8 * k + wave) * 1024), 16,
                                               wsrc[k], wstep * t, 0, 0);
  if (L::kMx && wave >= 4 && wave < 4 + L::kSDma)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr *)(base + L::kSOff + (wave - 4) * 256), 2, ssrc, 2 * t, 0,
                                             0);
#pragma unroll
  for (int k = 0; k < L::kXDma; ++k)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr *)(base + (8 * k + wave) * 1024), 16, xsrc[k], 128 * t, 0,
                                             0);
}

template <int FMT, int STAGES, int BM>
__global__ __launch_bounds__(kThreads, 1) void qgemm_ks_kernel(float *__restrict__ out,
                                                               const uint16_t *__restrict__ X,
                                                               const uint8_t *__restrict__ Wq,
                                                               const void *__restrict__ scales, int M, int N,
                                                               int K) {
  using L = Layout<FMT, STAGES, BM>;
  __shared__ __attribute__((aligned(1024))) unsigned char lds[L::kLds];
  int tile = blockIdx.x;
  const int tiles = gridDim.x;
  if (tiles % kXcds == 0) tile = (tile % kXcds) * (tiles / kXcds) + tile / kXcds;
  const int mtiles = (M + L::kBM - 1) / L::kBM;
  const int m0 = (tile % mtiles) * L::kBM, n0 = (tile / mtiles) * L::kBN;
  const int mrows = min(L::kBM, M - m0), nrows = min(L::kBN, N - n0);
  const int tid = threadIdx.x, lane = tid % L2C_WAVE;
  const int wave = __builtin_amdgcn_readfirstlane(tid / L2C_WAVE);
  const int g = wave >> 2, p = wave & 3;
  const int wm = p % L::kWavesM, wn = p / L::kWavesM;
  const int r = lane % 32, h = lane / 32;
  const int xrb = 2 * K;
  const int wrb = L::kMx ? K / 2 : K;
  const int srb = K / 32;
  const __amdgpu_buffer_rsrc_t rx =
      l2c::buffer_rsrc(X + static_cast<size_t>(m0) * K, static_cast<uint32_t>(mrows) * xrb);
  const __amdgpu_buffer_rsrc_t rw =
      l2c::buffer_rsrc(Wq + static_cast<size_t>(n0) * wrb, static_cast<uint32_t>(nrows) * wrb);
  const __amdgpu_buffer_rsrc_t rs =
      L::kMx ? l2c::buffer_rsrc(static_cast<const uint8_t *>(scales) + static_cast<size_t>(n0) * srb,
                                static_cast<uint32_t>(nrows) * srb)
             : rw;

  // DMA sources (per-lane parts; the step's k offset is scalar). X: block b of
  // 8 rows (b = 8k + wave, k < BM / 64), lane i fills row 8b + i / 8, slot
  // i % 8 with chunk (i % 8) ^ xswizzle(row). W: instruction q = 8k + wave
  // (while q < kWDma) fills rows (64 / lanes-per-row) q + i / lanes-per-row,
  // slot i % lanes-per-row. MXFP4 scales: wave 4 + s fills row 64 s + i.
  const int lrow = 8 * wave + lane / 8;
  const int lchunk = 16 * ((lane % 8) ^ xswizzle(lrow));
  int xsrc[4] = {0, 0, 0, 0};
#pragma unroll
  for (int k = 0; k < L::kXDma; ++k) xsrc[k] = min(64 * k + lrow, mrows - 1) * xrb + lchunk;
  int wsrc[2] = {0, 0};
#pragma unroll
  for (int k = 0; k < (L::kWDma + 7) / 8; ++k) {
    const int wrow = L::kWRowsPerDma * (8 * k + wave) + lane / L::kLanesPerRow;
    wsrc[k] = min(wrow, nrows - 1) * wrb + 16 * ((lane % L::kLanesPerRow) ^ L::wswizzle(wrow));
  }
  const int ssrc = min(max(64 * (wave - 4) + lane, 0), nrows - 1) * srb;
  const int wstep = L::kWRow;
  auto dma = [&](int stage, int t) __attribute__((always_inline)) {
    issue_step_dma<FMT, STAGES, BM>(lds + stage * L::kStage, t, wave, rx, rw, rs, xsrc, wsrc, ssrc, wstep);
  };
  // This wave's DMA of the step after the one just read has landed, its LDS
  // reads are done; then the workgroup barrier. The DMA of the STAGES - 2
  // newer steps may stay in flight (Layout::kWait instructions; one form for
  // every wave: no branch for the compiler to sink the conversions past).
  auto wait_dma_barrier = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (L::kWait == 8)
      asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else if constexpr (L::kWait == 6)
      asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else if constexpr (L::kWait == 4)
      asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
      static_assert(L::kWait == 8, "no wait form for this layout");
    __builtin_amdgcn_sched_barrier(0);
  };
  auto barrier = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // Fragments. X rows wm * 128 + 32 i + r, chunks 4h + 2g (+1). W rows
  // wn * 64 + 32 j + r (the swizzle of row + 32 equals that of row): MXFP4
  // bytes 16h + 8g of the 32-byte row (chunk h), fp8 bytes 32h + 16g (chunk
  // 2h + g); the MXFP4 scale word of the row (byte h is the lane's block).
  const int xsw = xswizzle(r);
  const int a0 = (wm * 128 + r) * 128;
  const int c0 = 16 * ((4 * h + 2 * g) ^ xsw), c1 = 16 * ((4 * h + 2 * g + 1) ^ xsw);
  const int wr0 = wn * 64 + r;
  const int wb = L::kMx ? L::kXBytes + wr0 * 32 + 16 * (h ^ L::wswizzle(wr0)) + 8 * g
                        : L::kXBytes + wr0 * 64 + 16 * ((2 * h + g) ^ L::wswizzle(wr0));
  const int sb = L::kSOff + 4 * wr0;
  u32x4 fa[4][2];
  u32x4 wc[2];
  uint32_t ws[2];
  auto read = [&](int stage) __attribute__((always_inline)) {
    const unsigned char *base = lds + stage * L::kStage;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if constexpr (L::kMx) {
        const u32x2 v = *reinterpret_cast<const u32x2 *>(base + wb + 1024 * j);
        wc[j][0] = v[0], wc[j][1] = v[1];
        ws[j] = *reinterpret_cast<const uint32_t *>(base + sb + 128 * j);
      } else {
        wc[j] = *reinterpret_cast<const u32x4 *>(base + wb + 2048 * j);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[i][0] = *reinterpret_cast<const u32x4 *>(base + a0 + 4096 * i + c0);
      fa[i][1] = *reinterpret_cast<const u32x4 *>(base + a0 + 4096 * i + c1);
    }
  };
  bf16x8 b[2][2];
  auto convert = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        uint32_t d[4];
        if constexpr (L::kMx) {
          // The block's scale byte h as an fp32 exponent field: the
          // conversion reads only that field, so scale byte 0 (0.0f) scales
          // by 2^-127, its E8M0 value.
          const float scale = __uint_as_float(((ws[j] >> (8 * h)) & 0xffu) << 23);
          const uint32_t c = wc[j][q];
          d[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, scale, 0));
          d[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, scale, 1));
          d[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, scale, 2));
          d[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, scale, 3));
        } else {
          const uint32_t c0w = wc[j][2 * q], c1w = wc[j][2 * q + 1];
          d[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c0w, 1.0f, false));
          d[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c0w, 1.0f, true));
          d[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c1w, 1.0f, false));
          d[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c1w, 1.0f, true));
        }
        b[j][q] = __builtin_bit_cast(bf16x8, make_uint4(d[0], d[1], d[2], d[3]));
      }
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
#pragma unroll
  for (int st = 0; st < STAGES - 1; ++st) dma(st, min(st, last));
  wait_dma_barrier();  // step 0 landed everywhere
  if (g == 1) barrier();
  int cur = 0;
  for (int t = 0; t < total; ++t) {
    // Memory phase of step t: the fragment reads go first, then the DMA of
    // step t + STAGES - 1 into the stage step t - 1 held (both groups read it
    // before the last barrier), then the conversions.
    read(cur);
    dma(cur == 0 ? STAGES - 1 : cur - 1, min(t + STAGES - 1, last));
    convert();
    wait_dma_barrier();
    // MFMA phase of step t.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fa[i][c]), b[j][c],
                                                              acc[i][j], 0, 0, 0);
    __builtin_amdgcn_s_setprio(0);
    barrier();
    cur = cur == STAGES - 1 ? 0 : cur + 1;
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
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = wn * 64 + 32 * j + r;
      float rscale = 1.0f;
      if constexpr (!L::kMx) rscale = n < nrows ? static_cast<const float *>(scales)[n0 + n] : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int m = wm * 128 + 32 * i + 8 * (v / 4) + 4 * h + v % 4;
          const float sum = acc[i][j][v] + exchange[((p * 8 + i * 2 + j) * 16 + v) * L2C_WAVE + lane];
          // Nontemporal: the tile's outputs are written once, at the end of
          // the launch, when every CU stores at once (fp8 198.2-198.6 against
          // 199.9-200.7 µs with ordinary stores, MXFP4 200.8-201.1 against
          // 202.2-202.5, at 1024 x 16384 x 8192 on one box).
          if (m < mrows && n < nrows)
            __builtin_nontemporal_store(sum * rscale, &out[static_cast<size_t>(m0 + m) * N + n0 + n]);
        }
    }
  }
}

}  // namespace

namespace {
// MXFP4 takes 256 x 128 tiles, fp8 128 x 256 (same time alone, and its four
// 32 KB stages leave LDS for the row kernels beside it in an iteration).
int tile_rows(int fmt) { return fmt == L2C_Q_MXFP4 ? 256 : 128; }
}  // namespace

long long l2c_qgemm_ks_tiles(int fmt, int batch, int rows) {
  const int bm = tile_rows(fmt), bn = 32768 / bm;
  return static_cast<long long>((batch + bm - 1) / bm) * ((rows + bn - 1) / bn);
}

// Called by l2c_matmul_q after its argument checks, for cols % 64 == 0 (and,
// for MXFP4, scales at an even address: the scale DMAs read 2 bytes).
int l2c_matmul_q_ks(float *out, const uint16_t *X, const uint8_t *Wq, const void *scales, int fmt, int batch,
                    int cols, int rows, hipStream_t stream) {
  if (cols % 64 != 0 || (fmt != L2C_Q_MXFP4 && fmt != L2C_Q_FP8)) return hipErrorInvalidValue;
  if (fmt == L2C_Q_MXFP4 && (reinterpret_cast<uintptr_t>(scales) & 1u)) return hipErrorInvalidValue;
  const int bm = tile_rows(fmt), bn = 32768 / bm;
  // Per-lane byte offsets are ints: a tile's X rows and W rows stay below 2^31.
  if (static_cast<long long>(bm) * cols * 2 > 0x7fffffffLL) return hipErrorInvalidValue;
  if (static_cast<long long>(bn) * (fmt == L2C_Q_MXFP4 ? cols / 2 : cols) > 0x7fffffffLL) return hipErrorInvalidValue;
  const long long tiles = l2c_qgemm_ks_tiles(fmt, batch, rows);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(tiles)), block(kThreads);
  // Four stages: 146 KB (MXFP4), 128 KB (fp8).
  if (fmt == L2C_Q_MXFP4)
    hipLaunchKernelGGL((qgemm_ks_kernel<L2C_Q_MXFP4, 4, 256>), grid, block, 0, stream, out, X, Wq, scales, batch,
                       rows, cols);
  else
    hipLaunchKernelGGL((qgemm_ks_kernel<L2C_Q_FP8, 4, 128>), grid, block, 0, stream, out, X, Wq, scales, batch, rows,
                       cols);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

int l2c_qgemm_ks_occupancy(int fmt, int *blocks_per_cu) {
  const void *fn = fmt == L2C_Q_MXFP4 ? reinterpret_cast<const void *>(qgemm_ks_kernel<L2C_Q_MXFP4, 4, 256>)
                                      : reinterpret_cast<const void *>(qgemm_ks_kernel<L2C_Q_FP8, 4, 128>);
  return static_cast<int>(hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, fn, kThreads, 0));
}
