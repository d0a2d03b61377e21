// Quantized-weight contraction out[b][r] = sum_k X[b][k] * deq(W)[r][k] with
// bf16 activations and MXFP4 or per-row-scaled fp8 e4m3 weights, plus the
// device quantizers that produce those weights.
//
// Kernel design (gfx950):
//  * The activations are bf16 and must stay bf16 (the oracle multiplies the
//    exact bf16 values), so the product runs on the bf16 matrix cores
//    (v_mfma_f32_32x32x16_bf16, fp32 accumulation).
//  * Weights are dequantized exactly to bf16 on their way into LDS, once per
//    workgroup and k-step: an e2m1 magnitude times a power of two, or an e4m3
//    value, has at most 4 significant bits, so the bf16 value is exact. The
//    fp8 row scale is applied once per output in the epilogue.
//  * Tile 256 (batch) x 128 (rows) x 64 (k), 8 wavefronts of 64 x 64, double-
//    buffered LDS with a 144-byte row stride (conflict-free 16-byte fragment
//    reads). MFMA operand layout: lane l supplies A[l % 32][8 * (l / 32) + 0..7]
//    and B[8 * (l / 32) + 0..7][l % 32]; the accumulator layout matches the
//    fp32 kernel's.
//  * Workgroup order is remapped per XCD as in the fp32 kernel.
//
// Encodings (bit-identical to the host encoders of the harness):
//  * e2m1: magnitudes {0, .5, 1, 1.5, 2, 3, 4, 6}, bit 3 the sign; nearest,
//    ties to the even code, saturating at 6, -0 -> +0. Two codes per byte,
//    even k in the low nibble. Block of 32 k: e8m0 scale 2^(s - 127) with
//    s - 127 = floor(log2(amax / 6)) clamped to [-127, 127].
//  * e4m3 (OCP, bias 7, max 448, no infinities): nearest-even, saturating.
#include "l2c_common.h"
#include "../../include/l2c.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

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

static_assert(kBN * (kBK / 16) == kThreads, "one 16-element weight chunk per thread");

struct Smem {
  uint16_t a[2][kBM][kStride];
  uint16_t b[2][kBN][kStride];
};

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

// bf16 bits of an e2m1 code times 2^x (exact: at most 2 significant bits).
__device__ __forceinline__ uint16_t e2m1_to_bf16(unsigned code, float scale) {
  constexpr float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  float v = mag[code & 7u] * scale;
  if (code & 8u) v = -v;
  return static_cast<uint16_t>(__float_as_uint(v) >> 16);
}

// bf16 bits of an e4m3 code (exact).
__device__ __forceinline__ uint16_t e4m3_to_bf16(unsigned code) {
  const unsigned e = (code >> 3) & 15u, m = code & 7u;
  unsigned bits;
  if (e == 0) bits = __float_as_uint(static_cast<float>(m) * 0.001953125f);  // m * 2^-9
  else bits = ((e + 120u) << 23) | (m << 20);
  bits |= (code & 0x80u) << 24;
  return static_cast<uint16_t>(bits >> 16);
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
  __shared__ Smem sm;
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

  // This thread's weight chunk: 16 consecutive k of one row.
  const int wrow = t / (kBK / 16);
  const int wchunk = t % (kBK / 16);
  const int wr = n0 + wrow;

  uint4 gx[kXChunks];
  uint4 gw;        // raw codes: 8 bytes (mxfp4, in .x/.y) or 16 bytes (fp8)
  unsigned gs = 0; // mxfp4 scale byte

  auto global_load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < kXChunks; ++i) {
      const int idx = t + i * kThreads;
      const int row = m0 + idx / (kBK / 8);
      const int k = k0 + (idx % (kBK / 8)) * 8;
      gx[i] = (row < M && k < K)
                  ? *reinterpret_cast<const uint4 *>(X + static_cast<size_t>(row) * K + k)
                  : make_uint4(0, 0, 0, 0);
    }
    const int k = k0 + wchunk * 16;
    const bool ok = wr < N && k < K;
    if constexpr (FMT == L2C_Q_MXFP4) {
      if (ok) {
        const uint2 c = *reinterpret_cast<const uint2 *>(Wq + static_cast<size_t>(wr) * (K / 2) + k / 2);
        gw = make_uint4(c.x, c.y, 0, 0);
        gs = static_cast<const uint8_t *>(scales)[static_cast<size_t>(wr) * (K / 32) + k / 32];
      } else {
        gw = make_uint4(0, 0, 0, 0);
        gs = 127;
      }
    } else {
      gw = ok ? *reinterpret_cast<const uint4 *>(Wq + static_cast<size_t>(wr) * K + k)
              : make_uint4(0, 0, 0, 0);
    }
  };

  auto lds_store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kXChunks; ++i) {
      const int idx = t + i * kThreads;
      *reinterpret_cast<uint4 *>(&sm.a[buf][idx / (kBK / 8)][(idx % (kBK / 8)) * 8]) = gx[i];
    }
    uint32_t h[8];  // 16 bf16, two per word
    if constexpr (FMT == L2C_Q_MXFP4) {
      // 2^(gs - 127); gs = 0 is the subnormal 2^-127.
      const float scale = gs == 0 ? __uint_as_float(0x00400000u) : pow2f(static_cast<int>(gs) - 127);
      const uint32_t words[2] = {gw.x, gw.y};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t w = words[i / 4];
        const unsigned lo = (w >> (8 * (i % 4))) & 15u, hi = (w >> (8 * (i % 4) + 4)) & 15u;
        h[i] = e2m1_to_bf16(lo, scale) | (static_cast<uint32_t>(e2m1_to_bf16(hi, scale)) << 16);
      }
    } else {
      const uint32_t words[4] = {gw.x, gw.y, gw.z, gw.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t w = words[i / 2];
        const unsigned lo = (w >> (16 * (i % 2))) & 0xffu, hi = (w >> (16 * (i % 2) + 8)) & 0xffu;
        h[i] = e4m3_to_bf16(lo) | (static_cast<uint32_t>(e4m3_to_bf16(hi)) << 16);
      }
    }
    uint4 *dst = reinterpret_cast<uint4 *>(&sm.b[buf][wrow][wchunk * 16]);
    dst[0] = make_uint4(h[0], h[1], h[2], h[3]);
    dst[1] = make_uint4(h[4], h[5], h[6], h[7]);
  };

  f32x16 acc[kFragM][kFragN];
#pragma unroll
  for (int i = 0; i < kFragM; ++i)
#pragma unroll
    for (int j = 0; j < kFragN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int frag_row = lane % 32;
  const int frag_k = 8 * (lane / 32);
  const int nk = (K + kBK - 1) / kBK;

  global_load(0);
  lds_store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) global_load((kt + 1) * kBK);
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 16) {
      bf16x8 a[kFragM], b[kFragN];
#pragma unroll
      for (int i = 0; i < kFragM; ++i)
        a[i] = *reinterpret_cast<const bf16x8 *>(&sm.a[buf][wm * kWaveM + i * 32 + frag_row][kk + frag_k]);
#pragma unroll
      for (int j = 0; j < kFragN; ++j)
        b[j] = *reinterpret_cast<const bf16x8 *>(&sm.b[buf][wn * kWaveN + j * 32 + frag_row][kk + frag_k]);
#pragma unroll
      for (int i = 0; i < kFragM; ++i)
#pragma unroll
        for (int j = 0; j < kFragN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) lds_store(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < kFragN; ++j) {
    const int n = n0 + wn * kWaveN + j * 32 + lane % 32;
    float rs = 1.0f;
    if constexpr (FMT == L2C_Q_FP8) rs = n < N ? static_cast<const float *>(scales)[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < kFragM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * kWaveM + i * 32 + 8 * (v / 4) + 4 * (lane / 32) + v % 4;
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
