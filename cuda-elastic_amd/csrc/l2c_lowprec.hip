// Device quantizers of the low-precision classifier cases: MXFP6 (E3M2 with
// UE8M0 scales per 32 values), NVFP4 (E2M1 with UE4M3 scales per 16 values
// and FP32 tensor scales) and BF16
// (experiments/blackwell/lowprec/spec.json "mxfp6", "nvfp4", "layout";
// the reference's kernels are decoder_lowprec.cu:202-340).
//
// Layouts (row-major [rows][width], width along K):
//  * MXFP6: the tiled operand layout of the MXFP6 contraction (rows padded
//    to Rp, a multiple of 32; padding rows hold zero codes and scales):
//      codes  [width / 128][Rp / 32][4 blocks][32 rows][24 B]
//      scales [width / 128][Rp][4 B]  (byte b = block b of the 128-value step)
//    24 B are one 32-value block's E3M2 codes as a little-endian bit stream
//    (value i at bits 6i..6i+5), the spec's packing; the reference keeps whole
//    rows contiguous and its scales in CUTLASS's tile layout for its GEMM. The
//    byte values are the same; only their order differs.
//  * NVFP4 codes: two per byte, even index in the low nibble, [rows][width / 2].
//    Scales: [rows][width / 16] UE4M3 bytes. Tensor scales: s = 2688 / a_t
//    (1 when a_t = 0) and d = 1 / s, both FP32.
//  * NVFP4 bf16 expansion (optional): [rows][width] bf16 of each element's
//    value times its block scale (d apart). The product of an E2M1 magnitude
//    (at most 2 significant bits) and a UE4M3 value (at most 4) has at most 6
//    significant bits and lies in [2^-10, 2688], so the bf16 value is exact:
//    it is the operand form the bf16 matrix cores multiply.
//
// Every quantizer reads its input once, coalesced. MXFP6: two lanes a block,
// 16 consecutive floats each, one workgroup per 3 KB output tile. NVFP4: one
// lane a 16-value block.
#include "l2c_common.h"
#include "l2c_formats.h"
#include "../../include/l2c.h"

namespace {

constexpr int kThreads = 256;
typedef float f32x2 __attribute__((ext_vector_type(2)));
constexpr int kAmaxBlocks = 1024;  // partial maxima of the tensor-scale pass

// One workgroup per output tile: k-step t (128 values) of the 32 rows of
// group g, whose codes are 3 KB contiguous in the tiled layout (block b of row
// r at byte (b * 32 + r) * 24) and whose scale words are 128 B contiguous.
// Thread i takes half h = i % 2 of block b = (i / 2) % 4 of row r = i / 8:
// 16 values, read as 64 contiguous bytes (the 8 threads of a row read its
// 512 bytes side by side). The block maximum is one shuffle between the two
// halves; a half's 16 codes are exactly dwords 3h .. 3h + 2 of the block's
// 24-byte stream (value i at bits 6i .. 6i + 5). Rows past `rows` are
// padding: zero codes and scale.
__global__ __launch_bounds__(kThreads) void quantize_mxfp6_kernel(uint8_t *__restrict__ codes,
                                                                  uint8_t *__restrict__ scales,
                                                                  const float *__restrict__ x, int rows,
                                                                  int width) {
  const int Rp = (rows + 31) / 32 * 32;
  const int groups = Rp / 32;
  const int t = static_cast<int>(blockIdx.x) / groups, g = static_cast<int>(blockIdx.x) % groups;
  const int i = threadIdx.x;
  const int r = i >> 3, b = (i >> 1) & 3, h = i & 1;
  const int row = g * 32 + r;
  float v[16];
  if (row < rows) {
    const float4 *src = reinterpret_cast<const float4 *>(x + static_cast<size_t>(row) * width + t * 128 + b * 32 +
                                                         h * 16);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 q = src[c];
      v[4 * c] = q.x, v[4 * c + 1] = q.y, v[4 * c + 2] = q.z, v[4 * c + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = 0.0f;
  }
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < 16; ++k) amax = fmaxf(amax, fabsf(v[k]));
  amax = fmaxf(amax, __shfl_xor(amax, 1, L2C_WAVE));
  const int X = l2c::mxfp6_exponent(amax);
  const float inv = l2c::pow2_neg(X);
  unsigned w[3] = {0u, 0u, 0u};
  if (amax > 0.0f) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const unsigned c = l2c::e3m2_code(v[k] * inv);
      const int pos = 6 * k, word = pos / 32, sh = pos % 32;
      w[word] |= c << sh;
      if (sh > 26) w[word + 1] |= c >> (32 - sh);
    }
  }
  const size_t tile = static_cast<size_t>(t) * groups + g;
  unsigned *dst = reinterpret_cast<unsigned *>(codes + tile * 3072 + (b * 32 + r) * 24 + h * 12);
  dst[0] = w[0], dst[1] = w[1], dst[2] = w[2];
  if (h == 0) scales[(static_cast<size_t>(t) * Rp + row) * 4 + b] = amax > 0.0f ? static_cast<uint8_t>(X + 127) : 0;
}

// Partial maxima of |x| over a grid-stride walk; one per workgroup.
__global__ __launch_bounds__(kThreads) void amax_partials_kernel(float *__restrict__ partials,
                                                                 const float *__restrict__ x,
                                                                 long long n) {
  __shared__ float slots[kThreads / L2C_WAVE];
  float m = 0.0f;
  const long long n4 = n / 4;
  const long long stride = static_cast<long long>(gridDim.x) * kThreads;
  for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < n4; i += stride) {
    const float4 v = reinterpret_cast<const float4 *>(x)[i];
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  for (long long i = 4 * n4 + static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride)
    m = fmaxf(m, fabsf(x[i]));
  m = l2c::block_max(m, slots);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

// The tensor maximum from the partials, then s = 2688 / a_t (1 for a_t = 0),
// d = 1 / s, and alpha = d * other_decode when asked (FP32, IEEE division).
__global__ __launch_bounds__(kThreads) void nvfp4_scales_kernel(float *__restrict__ tensor_scales,
                                                                float *__restrict__ alpha,
                                                                const float *__restrict__ other_decode,
                                                                const float *__restrict__ partials,
                                                                int count) {
#pragma clang fp contract(off)
  __shared__ float slots[kThreads / L2C_WAVE];
  float m = 0.0f;
  for (int i = threadIdx.x; i < count; i += kThreads) m = fmaxf(m, partials[i]);
  m = l2c::block_max(m, slots);
  if (threadIdx.x == 0) {
    const float s = l2c::nvfp4_encode_scale(m);
    const float d = 1.0f / s;
    tensor_scales[0] = s;
    tensor_scales[1] = d;
    if (alpha) *alpha = d * *other_decode;
  }
}

// The same scales from a tensor maximum already held as float bits in
// `absmax` (l2c_decoder_rmsnorm_absmax's), which is then cleared for the
// next maximum. One lane.
__global__ void nvfp4_scales_absmax_kernel(float *__restrict__ tensor_scales, float *__restrict__ alpha,
                                           const float *__restrict__ other_decode, unsigned *__restrict__ absmax) {
#pragma clang fp contract(off)
  const float m = __uint_as_float(*absmax);
  const float s = l2c::nvfp4_encode_scale(m);
  const float d = 1.0f / s;
  tensor_scales[0] = s;
  tensor_scales[1] = d;
  if (alpha) *alpha = d * *other_decode;
  *absmax = 0u;
}

// Scale code UE4M3((a / 6) s), codes E2M1((v s) / f), each step an FP32
// operation in this order; a zero scale code zeroes the block. Optionally also
// the exact bf16 values code * f. One lane per 16-value block: it reads the
// block's 64 bytes, takes the block maximum in registers and writes its 8 code
// bytes (element 2i in the low nibble of byte i), its scale byte and its 32
// bytes of bf16 expansion; consecutive lanes write consecutive blocks.
__global__ __launch_bounds__(kThreads) void quantize_nvfp4_kernel(uint8_t *__restrict__ codes,
                                                                  uint8_t *__restrict__ scales,
                                                                  uint16_t *__restrict__ expanded,
                                                                  const float *__restrict__ x,
                                                                  const float *__restrict__ tensor_scales,
                                                                  long long blocks) {
#pragma clang fp contract(off)
  const long long blk = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (blk >= blocks) return;
  const float4 *src = reinterpret_cast<const float4 *>(x) + blk * 4;
  float e[16];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 v = src[q];
    e[4 * q] = v.x, e[4 * q + 1] = v.y, e[4 * q + 2] = v.z, e[4 * q + 3] = v.w;
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(e[i]));
  const float s = tensor_scales[0];
  const unsigned sc = l2c::nvfp4_scale_code(amax, s);
  const float f = l2c::ue4m3_value(sc);
  // E2M1((v s) / f), the two steps in this order, by the hardware conversion
  // at scale 1 (nearest-even, saturating at 6): it gives e2m1_code's code for
  // every value but the negative ones that round to zero, where it keeps the
  // sign; those become +0 below. Two codes a conversion, packed into byte k
  // of the word (element 2k in the low nibble). A zero scale code zeroes the
  // block (f is 0 there, so the quotients are not finite).
  float r[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float t = e[i] * s;
    r[i] = t / f;
  }
  unsigned lo = 0, hi = 0;
  lo = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(lo, r[0], r[1], 1.0f, 0);
  lo = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(lo, r[2], r[3], 1.0f, 1);
  lo = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(lo, r[4], r[5], 1.0f, 2);
  lo = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(lo, r[6], r[7], 1.0f, 3);
  hi = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(hi, r[8], r[9], 1.0f, 0);
  hi = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(hi, r[10], r[11], 1.0f, 1);
  hi = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(hi, r[12], r[13], 1.0f, 2);
  hi = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(hi, r[14], r[15], 1.0f, 3);
  auto positive_zeros = [](unsigned w) {
    const unsigned nonzero = ((w & 0x77777777u) + 0x77777777u) & 0x88888888u;  // 8 where magnitude != 0
    return w & (nonzero | 0x77777777u);
  };
  lo = sc != 0 ? positive_zeros(lo) : 0u;
  hi = sc != 0 ? positive_zeros(hi) : 0u;
  reinterpret_cast<uint2 *>(codes)[blk] = make_uint2(lo, hi);
  scales[blk] = static_cast<uint8_t>(sc);
  if (expanded) {
    // code * f, exact: an E2M1 value (at most 2 significant bits) times a
    // UE4M3 value (at most 4) has at most 6, so its bf16 is its top half.
    const f32x2 v[8] = {__builtin_amdgcn_cvt_scalef32_pk_f32_fp4(lo, 1.0f, 0),
                        __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(lo, 1.0f, 1),
                        __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(lo, 1.0f, 2),
                        __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(lo, 1.0f, 3),
                        __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(hi, 1.0f, 0),
                        __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(hi, 1.0f, 1),
                        __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(hi, 1.0f, 2),
                        __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(hi, 1.0f, 3)};
    unsigned b[16];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      b[2 * k] = __float_as_uint(v[k][0] * f) >> 16;
      b[2 * k + 1] = __float_as_uint(v[k][1] * f) >> 16;
    }
    uint4 *dst = reinterpret_cast<uint4 *>(expanded) + blk * 2;
    dst[0] = make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16));
    dst[1] = make_uint4(b[8] | (b[9] << 16), b[10] | (b[11] << 16), b[12] | (b[13] << 16), b[14] | (b[15] << 16));
  }
}

// BF16 round to nearest even, four values a thread (finite values never
// round to infinity: reference.cpp:84-96 picks between the truncation and the
// next finite magnitude).
__device__ __forceinline__ unsigned bf16_rne(float f) {
  const unsigned bits = __float_as_uint(f);
  if ((bits & 0x7f800000u) == 0x7f800000u) return bits >> 16;
  unsigned r = (bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16;
  if ((r & 0x7fffu) == 0x7f80u) --r;
  return r;
}

__global__ __launch_bounds__(kThreads) void to_bf16_x4_kernel(uint2 *__restrict__ out,
                                                              const float4 *__restrict__ in,
                                                              long long n4) {
  const long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n4) return;
  const float4 v = in[i];
  out[i] = make_uint2(bf16_rne(v.x) | (bf16_rne(v.y) << 16), bf16_rne(v.z) | (bf16_rne(v.w) << 16));
}

bool grid_ok(long long threads, unsigned *grid) {
  const long long g = (threads + kThreads - 1) / kThreads;
  if (g > 0x7fffffffLL) return false;
  *grid = static_cast<unsigned>(g);
  return true;
}

}  // namespace

extern "C" int l2c_quantize_mxfp6(uint8_t *codes, uint8_t *scales, const float *x, int rows, int width,
                                  hipStream_t stream) {
  if (rows < 0 || width <= 0 || width % 128 != 0) return hipErrorInvalidValue;
  if (rows == 0) return hipSuccess;
  if (!codes || !scales || !x || !l2c_aligned16(x) || (reinterpret_cast<uintptr_t>(codes) & 3u))
    return hipErrorInvalidValue;
  const long long tiles = static_cast<long long>((rows + 31) / 32) * (width / 128);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(quantize_mxfp6_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, stream, codes,
                     scales, x, rows, width);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

extern "C" int l2c_nvfp4_tensor_scales(float *tensor_scales, float *alpha, const float *other_decode,
                                       const float *x, long long n, float *partials, hipStream_t stream) {
  if (n < 0 || !tensor_scales || !partials || (n > 0 && !x) || (alpha && !other_decode))
    return hipErrorInvalidValue;
  if (x && !l2c_aligned16(x)) return hipErrorInvalidValue;
  const long long want = (n / 4 + kThreads - 1) / kThreads;
  const int parts = static_cast<int>(want < 1 ? 1 : want > kAmaxBlocks ? kAmaxBlocks : want);
  hipLaunchKernelGGL(amax_partials_kernel, dim3(parts), dim3(kThreads), 0, stream, partials, x, n);
  L2C_LAUNCH_CHECK();
  hipLaunchKernelGGL(nvfp4_scales_kernel, dim3(1), dim3(kThreads), 0, stream, tensor_scales, alpha,
                     other_decode, static_cast<const float *>(partials), parts);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

extern "C" int l2c_nvfp4_tensor_scales_absmax(float *tensor_scales, float *alpha, const float *other_decode,
                                              unsigned *absmax_bits, hipStream_t stream) {
  if (!tensor_scales || !absmax_bits || (alpha && !other_decode)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(nvfp4_scales_absmax_kernel, dim3(1), dim3(1), 0, stream, tensor_scales, alpha, other_decode,
                     absmax_bits);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

extern "C" int l2c_quantize_nvfp4(uint8_t *codes, uint8_t *scales, uint16_t *expanded_bf16, const float *x,
                                  const float *tensor_scales, int rows, int width, hipStream_t stream) {
  if (rows < 0 || width <= 0 || width % 16 != 0) return hipErrorInvalidValue;
  if (rows == 0) return hipSuccess;
  if (!codes || !scales || !x || !tensor_scales || !l2c_aligned16(x) || (reinterpret_cast<uintptr_t>(codes) & 7u) ||
      (expanded_bf16 && !l2c_aligned16(expanded_bf16)))
    return hipErrorInvalidValue;
  const long long blocks = static_cast<long long>(rows) * (width / 16);
  unsigned grid;
  if (!grid_ok(blocks, &grid)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(quantize_nvfp4_kernel, dim3(grid), dim3(kThreads), 0, stream, codes, scales, expanded_bf16,
                     x, tensor_scales, blocks);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}

// The vectorized form of l2c_to_bf16 (l2c_qgemm.hip) for 16-byte aligned
// inputs whose length is a multiple of 4.
extern "C" int l2c_to_bf16_x4(uint16_t *out, const float *in, long long n, hipStream_t stream) {
  if (n < 0 || n % 4 != 0) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  if (!out || !in || !l2c_aligned16(in) || (reinterpret_cast<uintptr_t>(out) & 7u)) return hipErrorInvalidValue;
  unsigned grid;
  if (!grid_ok(n / 4, &grid)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(to_bf16_x4_kernel, dim3(grid), dim3(kThreads), 0, stream, reinterpret_cast<uint2 *>(out),
                     reinterpret_cast<const float4 *>(in), n / 4);
  L2C_LAUNCH_CHECK();
  return hipSuccess;
}
