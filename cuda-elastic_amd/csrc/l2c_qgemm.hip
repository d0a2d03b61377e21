// Quantized-weight contraction out[b][r] = sum_k X[b][k] * deq(W)[r][k] with
// bf16 activations and MXFP4 or per-row-scaled fp8 e4m3 weights, plus the
// device quantizers that produce those weights.
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
//    blocks of 32 x 32). Only the activations use LDS: a double-buffered slab
//    with a 144-byte row stride (conflict-free 16-byte fragment reads). W never
//    touches LDS: each wavefront loads the codes of its own 64 rows from
//    global memory (L2) into registers and converts them into MFMA B operands.
//  * Two steps of prefetch: the X slab and the W codes of step t + 2 are
//    loaded while step t multiplies, so the 0.5 us of MFMA work per step does
//    not wait for L2 latency. Register sets alternate with the step's parity.
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
constexpr int kWaveM = kBM / kWavesM;
constexpr int kWaveN = kBN / kWavesN;
constexpr int kFragM = kWaveM / 32;
constexpr int kFragN = kWaveN / 32;
constexpr int kStride = kBK + 8;  // bf16 per LDS row (144 bytes)
constexpr int kXChunks = kBM * (kBK / 8) / kThreads;  // 16-byte X chunks per thread: 4
constexpr int kXcds = 8;

constexpr int kSteps = kBK / 16;  // MFMAs per 32 x 32 block and k-step (4)

static_assert(kBK == 64, "the k permutation gives each lane half 32 consecutive k per step");

// ---------------------------------------------------------------------------
// Element encoders / decoders.

__device__ __forceinline__ unsigned e2m1_code(float v) {
  const float t = fabsf(v);
  unsigned c;
  if (t <= 0.25f) c = 0;
  else if (t < 0.75f) c = 1;
  else if (t <= 1.25f) c = 2;
  else if (t < 1.75f) c = 3;
  else if (t <= 2.5f) c = 4;
  else if (t < 3.5f) c = 5;
  else if (t <= 5.0f) c = 6;
  else c = 7;
  return (c != 0 && v < 0.0f) ? (c | 8u) : c;
}

__device__ __forceinline__ unsigned e4m3_code(float v) {
  const float a = fabsf(v);
  unsigned c;
  if (a < 0.015625f) {  // below 2^-6: subnormal codes m * 2^-9, m in 0..8
    c = static_cast<unsigned>(rintf(a * 512.0f));
  } else {
    const unsigned bits = __float_as_uint(a);
    int e = static_cast<int>((bits >> 23) & 0xffu) - 127;
    unsigned q = (bits >> 20) & 7u;
    const unsigned rem = bits & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) ++q;
    if (q == 8u) {
      q = 0;
      ++e;
    }
    c = e > 8 ? 0x7eu : ((static_cast<unsigned>(e + 7) << 3) | q);
    if (c > 0x7eu) c = 0x7eu;
  }
  return (c != 0 && v < 0.0f) ? (c | 0x80u) : c;
}

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
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][kBM][kStride];
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
  const int r = lane % 32;
  const int h = lane / 32;
  const int nk = (K + kBK - 1) / kBK;

  // X slab. Loads are clamped into the operand and used as loaded: rows past
  // M only feed outputs that are never stored, and k past K meets W codes
  // zeroed when the B operand is formed (finite x times 0 is 0).
  u32x4 gx[2][kXChunks];
  auto x_load = [&](u32x4 (&g)[kXChunks], int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kXChunks; ++i) {
      const int idx = t + i * kThreads;
      const int row = m0 + idx / (kBK / 8);
      const int k = k0 + (idx % (kBK / 8)) * 8;
      g[i] = *reinterpret_cast<const u32x4 *>(
          X + static_cast<size_t>(row < M ? row : M - 1) * K + (k < K ? k : K - 8));
    }
  };
  auto x_store = [&](const u32x4 (&g)[kXChunks], int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kXChunks; ++i) {
      const int idx = t + i * kThreads;
      *reinterpret_cast<u32x4 *>(&xs[buf][idx / (kBK / 8)][(idx % (kBK / 8)) * 8]) = g[i];
    }
  };

  // This lane's W row in each 32-row block and its codes for one step.
  int wrow[kFragN];
#pragma unroll
  for (int j = 0; j < kFragN; ++j) {
    const int n = n0 + wn * kWaveN + j * 32 + r;
    wrow[j] = n < N ? n : N - 1;
  }
  // Raw codes are kept exactly as loaded (no arithmetic on a load result
  // until it is used two steps later, so the loads stay in flight); rows past
  // N read a clamped row whose outputs are never stored, and k past K is
  // zeroed when the operand is formed.
  constexpr int kWords = FMT == L2C_Q_MXFP4 ? 4 : 8;  // dwords of codes per block and step
  uint32_t raw[2][kFragN][kWords];
  uint32_t sraw[2][kFragN];  // MXFP4 scale bytes as loaded
  bool kin[2];               // this lane half's k range lies inside K
  auto w_load = [&](uint32_t (&rw)[kFragN][kWords], uint32_t (&sr)[kFragN], bool &kok,
                    int k0) __attribute__((always_inline)) {
    const int k = k0 + 32 * h;
    kok = k < K;
    const int kc = kok ? k : K - 32;
#pragma unroll
    for (int j = 0; j < kFragN; ++j) {
      if constexpr (FMT == L2C_Q_MXFP4) {
        const uint4 v =
            *reinterpret_cast<const uint4 *>(Wq + static_cast<size_t>(wrow[j]) * (K / 2) + kc / 2);
        rw[j][0] = v.x;
        rw[j][1] = v.y;
        rw[j][2] = v.z;
        rw[j][3] = v.w;
        sr[j] = static_cast<const uint8_t *>(scales)[static_cast<size_t>(wrow[j]) * (K / 32) + kc / 32];
      } else {
        const uint4 *p = reinterpret_cast<const uint4 *>(Wq + static_cast<size_t>(wrow[j]) * K + kc);
        const uint4 v0 = p[0], v1 = p[1];
        rw[j][0] = v0.x;
        rw[j][1] = v0.y;
        rw[j][2] = v0.z;
        rw[j][3] = v0.w;
        rw[j][4] = v1.x;
        rw[j][5] = v1.y;
        rw[j][6] = v1.z;
        rw[j][7] = v1.w;
      }
    }
  };
  // B operand of MFMA q for block j: W[k = 32h + 8q + 0..7] of row wrow[j].
  auto w_operand = [&](const uint32_t (&rw)[kFragN][kWords], const uint32_t (&sr)[kFragN],
                       bool kok, int j, int q) __attribute__((always_inline)) {
    uint32_t d[4];
    if constexpr (FMT == L2C_Q_MXFP4) {
      // Block scale 2^(s - 127) as fp32 (s = 0 is the subnormal 2^-127); 0
      // outside K, which zeroes the converted values.
      const uint32_t sc = sr[j] & 0xffu;
      const float scale = __uint_as_float(kok ? (sc == 0 ? 0x00400000u : (sc << 23)) : 0u);
      const uint32_t w = rw[j][q];  // codes k = 8q .. 8q + 7, two per byte
      d[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0));
      d[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1));
      d[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2));
      d[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3));
    } else {
      const uint32_t w0 = kok ? rw[j][2 * q] : 0u, w1 = kok ? rw[j][2 * q + 1] : 0u;
      d[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false));
      d[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true));
      d[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false));
      d[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true));
    }
    return __builtin_bit_cast(bf16x8, make_uint4(d[0], d[1], d[2], d[3]));
  };

  f32x16 acc[kFragM][kFragN];
#pragma unroll
  for (int i = 0; i < kFragM; ++i)
#pragma unroll
    for (int j = 0; j < kFragN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const uint16_t *a_base = &xs[0][wm * kWaveM + r][32 * h];
  constexpr int kBuf = kBM * kStride;

  // One k-step; its parity P names its LDS buffer and register sets.
  auto step = [&](auto parity, int kt) __attribute__((always_inline)) {
    constexpr int P = decltype(parity)::value;
    bf16x8 bop[kFragN][kSteps];
#pragma unroll
    for (int j = 0; j < kFragN; ++j)
#pragma unroll
      for (int q = 0; q < kSteps; ++q) bop[j][q] = w_operand(raw[P], sraw[P], kin[P], j, q);
    if (kt + 2 < nk) {  // step t + 2 into the registers just consumed
      x_load(gx[P], (kt + 2) * kBK);
      w_load(raw[P], sraw[P], kin[P], (kt + 2) * kBK);
    }
#pragma unroll
    for (int q = 0; q < kSteps; ++q) {
      bf16x8 a[kFragM];
#pragma unroll
      for (int i = 0; i < kFragM; ++i)
        a[i] = *reinterpret_cast<const bf16x8 *>(a_base + P * kBuf + i * 32 * kStride + 8 * q);
#pragma unroll
      for (int i = 0; i < kFragM; ++i)
#pragma unroll
        for (int j = 0; j < kFragN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bop[j][q], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) x_store(gx[P ^ 1], P ^ 1);  // the slab of step t + 1
    __syncthreads();
  };

  x_load(gx[0], 0);
  w_load(raw[0], sraw[0], kin[0], 0);
  if (nk > 1) {
    x_load(gx[1], kBK);
    w_load(raw[1], sraw[1], kin[1], kBK);
  }
  x_store(gx[0], 0);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    step(std::integral_constant<int, 0>(), kt);
    if (kt + 1 < nk) step(std::integral_constant<int, 1>(), kt + 1);
  }

#pragma unroll
  for (int j = 0; j < kFragN; ++j) {
    const int n = n0 + wn * kWaveN + j * 32 + r;
    float rs = 1.0f;
    if constexpr (FMT == L2C_Q_FP8) rs = n < N ? static_cast<const float *>(scales)[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < kFragM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * kWaveM + i * 32 + 8 * (v / 4) + 4 * h + v % 4;
        if (m < M && n < N) out[static_cast<size_t>(m) * N + n] = acc[i][j][v] * rs;
      }
    }
  }
}

}  // namespace

int l2c_qgemm_launch_shape(int fmt, int batch, int cols, int rows, int *grid, int *block,
                           int *blocks_per_cu) {
  (void)cols;
  if (fmt != L2C_Q_MXFP4 && fmt != L2C_Q_FP8) return hipErrorInvalidValue;
  *grid = ((batch + kBM - 1) / kBM) * ((rows + kBN - 1) / kBN);
  *block = kThreads;
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
  const long long tiles =
      static_cast<long long>((batch + kBM - 1) / kBM) * ((rows + kBN - 1) / kBN);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(tiles)), block(kThreads);
  const uint16_t *X = static_cast<const uint16_t *>(Xbf16);
  const uint8_t *W = static_cast<const uint8_t *>(Wq);
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
