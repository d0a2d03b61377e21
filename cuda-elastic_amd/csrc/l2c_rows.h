// Device code of the row operations (rmsnorm, softmax, one matrix row dotted
// with x), shared by the row kernels and the fused kernel.
//
// A T-lane workgroup holds a row in VGPRs: lane t owns chunk c = t + i*T for
// i < V, a float4 (VEC) or, for rows that are not 16-byte aligned, four
// scalars at elements t + (4i + s)*T. EXACT means T * V * 4 == size, so no
// lane needs a bounds check.
#pragma once

#include "l2c_common.h"

namespace l2c {

template <int V, bool VEC, bool EXACT>
struct Row {
  float4 x[V];

  __device__ __forceinline__ void load(const float *row, int size, float fill) {
    const int T = blockDim.x, t = threadIdx.x;
    if constexpr (VEC) {
      const float4 *row4 = reinterpret_cast<const float4 *>(row);
      const int cols4 = size >> 2;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const int c = t + i * T;
        if constexpr (EXACT) x[i] = row4[c];
        else x[i] = c < cols4 ? row4[c] : make_float4(fill, fill, fill, fill);
      }
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const int j0 = t + (4 * i) * T;
        x[i].x = j0 < size ? row[j0] : fill;
        x[i].y = j0 + T < size ? row[j0 + T] : fill;
        x[i].z = j0 + 2 * T < size ? row[j0 + 2 * T] : fill;
        x[i].w = j0 + 3 * T < size ? row[j0 + 3 * T] : fill;
      }
    }
  }

  // Stores x * scale * weight[j] (weight may be null: x * scale) for every
  // valid element j, with 16-byte nontemporal stores on the vector path.
  __device__ __forceinline__ void store_scaled(float *row, int size, float scale,
                                               const float *weight) const {
    const int T = blockDim.x, t = threadIdx.x;
    if constexpr (VEC) {
      float4 *row4 = reinterpret_cast<float4 *>(row);
      const float4 *w4 = reinterpret_cast<const float4 *>(weight);
      const int cols4 = size >> 2;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const int c = t + i * T;
        if (EXACT || c < cols4) {
          float4 r;
          if (weight != nullptr) {
            const float4 g = w4[c];
            r.x = x[i].x * scale * g.x;
            r.y = x[i].y * scale * g.y;
            r.z = x[i].z * scale * g.z;
            r.w = x[i].w * scale * g.w;
          } else {
            r.x = x[i].x * scale;
            r.y = x[i].y * scale;
            r.z = x[i].z * scale;
            r.w = x[i].w * scale;
          }
          st4_stream(row4 + c, r);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float v[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int j = t + (4 * i + s) * T;
          if (j < size) row[j] = weight != nullptr ? v[s] * scale * weight[j] : v[s] * scale;
        }
      }
    }
  }
};

// Row reductions and transforms on a loaded row. `slots` is LDS scratch for
// two block reductions (32 floats).

template <int V, bool VEC, bool EXACT>
__device__ __forceinline__ void rmsnorm_apply(Row<V, VEC, EXACT> &r, float *out, const float *weight,
                                              int size, float eps, float *slots) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    ss = fmaf(r.x[i].x, r.x[i].x, ss);
    ss = fmaf(r.x[i].y, r.x[i].y, ss);
    ss = fmaf(r.x[i].z, r.x[i].z, ss);
    ss = fmaf(r.x[i].w, r.x[i].w, ss);
  }
  ss = block_sum(ss, slots);
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(size) + eps);
  r.store_scaled(out, size, scale, weight);
}

// exp(t) for t <= 0 (softmax arguments x - max) on the hardware exp2
// (v_exp_f32), with Cody-Waite range reduction (W. J. Cody and W. Waite,
// Software Manual for the Elementary Functions, 1980): t = n ln2 + r with
// n = rint(t / ln2) and |r| <= ln2 / 2, r computed with a two-part ln2
// (16 + 24 bits) by fused multiply-adds, then exp(t) = 2^n * 2^(r / ln2).
// The argument of v_exp_f32 is within [-1/2, 1/2], so its rounding
// (2^-25 absolute) adds at most 1.8e-8 relative error to v_exp_f32's own
// (about 1 ulp); the result is exact scaling by 2^n (v_ldexp_f32). Arguments
// below -104 (results under the smallest float subnormal, including the
// -FLT_MAX padding of a partial row) return 0; NaN propagates.
__device__ __forceinline__ float exp_nonpositive(float t) {
  constexpr float kLog2e = 1.44269504088896340736f;
  constexpr float kLn2Hi = 0.693145751953125f;        // 16 significant bits
  constexpr float kLn2Lo = 1.42860682030941723212e-6f; // ln2 - kLn2Hi
  const float n = rintf(t * kLog2e);
  float r = fmaf(-n, kLn2Hi, t);
  r = fmaf(-n, kLn2Lo, r);
  const float e = ldexpf(__builtin_amdgcn_exp2f(r * kLog2e), static_cast<int>(n));
  return t < -104.0f ? 0.0f : e;
}

// softmax with a single block reduction: each wavefront exponentiates
// against its own maximum m_w and sums (s_w); the waves' (m_w, s_w) pairs
// meet once in LDS, every lane combines them in wave order into the row
// maximum M and S = sum_w s_w exp(m_w - M), and stores e * (exp(m_w - M) / S).
// One barrier per row instead of two; one extra rounding per element.
template <int V, bool VEC, bool EXACT>
__device__ __forceinline__ void softmax_apply_1r(Row<V, VEC, EXACT> &r, float *out, int size,
                                                 float *slots) {
  float m = -FLT_MAX;
#pragma unroll
  for (int i = 0; i < V; ++i)
    m = fmaxf(m, fmaxf(fmaxf(r.x[i].x, r.x[i].y), fmaxf(r.x[i].z, r.x[i].w)));
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    r.x[i].x = exp_nonpositive(r.x[i].x - m);
    r.x[i].y = exp_nonpositive(r.x[i].y - m);
    r.x[i].z = exp_nonpositive(r.x[i].z - m);
    r.x[i].w = exp_nonpositive(r.x[i].w - m);
    s += (r.x[i].x + r.x[i].y) + (r.x[i].z + r.x[i].w);
  }
  s = wave_sum(s);
  const int waves = blockDim.x / L2C_WAVE, w = threadIdx.x / L2C_WAVE;
  if (threadIdx.x % L2C_WAVE == 0) {
    slots[2 * w] = m;
    slots[2 * w + 1] = s;
  }
  __syncthreads();
  float M = -FLT_MAX;
  for (int k = 0; k < waves; ++k) M = fmaxf(M, slots[2 * k]);
  float S = 0.0f;
  // Not unrolled: the unrolled loop's overlapping exps took the 8-float4 row
  // kernel to 59 VGPRs; rolled it takes 54, and two waves of it (2 x 56
  // allocated) fit on a SIMD beside the block-scaled contraction's two
  // (2 x 200), so softmax rows run during that product. Same order of
  // operations, same results.
#pragma unroll 1
  for (int k = 0; k < waves; ++k) S += slots[2 * k + 1] * exp_nonpositive(slots[2 * k] - M);
  r.store_scaled(out, size, exp_nonpositive(m - M) / S, nullptr);
}

// Dot product of matrix row `row` with x by one wavefront: 64 lanes x 16 B =
// 1 KiB contiguous per load instruction, four independent loads in flight per
// lane, one wave reduction; lane 0 writes out[row]. NT selects nontemporal
// loads of the matrix (they keep it from evicting x from L2); ordinary loads
// let the MALL keep a matrix that fits it between launches. The standalone
// product and the fused iteration both call this, so their outputs agree bit
// for bit.
template <bool VEC, bool NT>
__device__ __forceinline__ void matvec_wave_row(float *out, const float *x, const float *W, int cols,
                                                int row, int lane) {
  const float *w = W + static_cast<size_t>(row) * cols;
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  if constexpr (VEC) {
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const int cols4 = cols >> 2;
    int c = lane;
    for (; c + 3 * L2C_WAVE < cols4; c += 4 * L2C_WAVE) {
      const float4 m0 = NT ? ld4_stream(w4 + c) : w4[c];
      const float4 m1 = NT ? ld4_stream(w4 + c + L2C_WAVE) : w4[c + L2C_WAVE];
      const float4 m2 = NT ? ld4_stream(w4 + c + 2 * L2C_WAVE) : w4[c + 2 * L2C_WAVE];
      const float4 m3 = NT ? ld4_stream(w4 + c + 3 * L2C_WAVE) : w4[c + 3 * L2C_WAVE];
      const float4 v0 = x4[c], v1 = x4[c + L2C_WAVE];
      const float4 v2 = x4[c + 2 * L2C_WAVE], v3 = x4[c + 3 * L2C_WAVE];
      a0 = fmaf(m0.x, v0.x, a0); a0 = fmaf(m0.y, v0.y, a0);
      a0 = fmaf(m0.z, v0.z, a0); a0 = fmaf(m0.w, v0.w, a0);
      a1 = fmaf(m1.x, v1.x, a1); a1 = fmaf(m1.y, v1.y, a1);
      a1 = fmaf(m1.z, v1.z, a1); a1 = fmaf(m1.w, v1.w, a1);
      a2 = fmaf(m2.x, v2.x, a2); a2 = fmaf(m2.y, v2.y, a2);
      a2 = fmaf(m2.z, v2.z, a2); a2 = fmaf(m2.w, v2.w, a2);
      a3 = fmaf(m3.x, v3.x, a3); a3 = fmaf(m3.y, v3.y, a3);
      a3 = fmaf(m3.z, v3.z, a3); a3 = fmaf(m3.w, v3.w, a3);
    }
    for (; c < cols4; c += L2C_WAVE) {
      const float4 m0 = NT ? ld4_stream(w4 + c) : w4[c];
      const float4 v0 = x4[c];
      a0 = fmaf(m0.x, v0.x, a0); a0 = fmaf(m0.y, v0.y, a0);
      a0 = fmaf(m0.z, v0.z, a0); a0 = fmaf(m0.w, v0.w, a0);
    }
  } else {
    int c = lane;
    for (; c + 3 * L2C_WAVE < cols; c += 4 * L2C_WAVE) {
      a0 = fmaf(__builtin_nontemporal_load(w + c), x[c], a0);
      a1 = fmaf(__builtin_nontemporal_load(w + c + L2C_WAVE), x[c + L2C_WAVE], a1);
      a2 = fmaf(__builtin_nontemporal_load(w + c + 2 * L2C_WAVE), x[c + 2 * L2C_WAVE], a2);
      a3 = fmaf(__builtin_nontemporal_load(w + c + 3 * L2C_WAVE), x[c + 3 * L2C_WAVE], a3);
    }
    for (; c < cols; c += L2C_WAVE) a0 = fmaf(__builtin_nontemporal_load(w + c), x[c], a0);
  }
  const float acc = wave_sum((a0 + a1) + (a2 + a3));
  if (lane == 0) out[row] = acc;
}

// Dot product of matrix row `row` with x by a pair of wavefronts (aligned
// rows): wavefront `part` (0 or 1) streams its contiguous half of the row's
// float4 chunks as matvec_wave_row streams a whole row; the two wave sums meet
// in `slots` (one float a wavefront of the workgroup) and part 0 adds part 1's
// to its own. Every wavefront of the workgroup must call it (it holds a
// workgroup barrier); `live` false does the barrier only. Measured at
// 8192 x 16384 against one wavefront a row: 82.0 against 84.0 us (one box).
template <bool NT>
__device__ __forceinline__ void matvec_pair_row(float *out, const float *x, const float *W, int cols, int row,
                                                int part, int lane, bool live, float *slots) {
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  if (live) {
    const int cols4 = cols >> 2, half = (cols4 + 1) >> 1;
    const int begin = part * half, end = part ? cols4 : half;
    const float4 *w4 = reinterpret_cast<const float4 *>(W + static_cast<size_t>(row) * cols);
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    int c = begin + lane;
    for (; c + 3 * L2C_WAVE < end; c += 4 * L2C_WAVE) {
      const float4 m0 = NT ? ld4_stream(w4 + c) : w4[c];
      const float4 m1 = NT ? ld4_stream(w4 + c + L2C_WAVE) : w4[c + L2C_WAVE];
      const float4 m2 = NT ? ld4_stream(w4 + c + 2 * L2C_WAVE) : w4[c + 2 * L2C_WAVE];
      const float4 m3 = NT ? ld4_stream(w4 + c + 3 * L2C_WAVE) : w4[c + 3 * L2C_WAVE];
      const float4 v0 = x4[c], v1 = x4[c + L2C_WAVE];
      const float4 v2 = x4[c + 2 * L2C_WAVE], v3 = x4[c + 3 * L2C_WAVE];
      a0 = fmaf(m0.x, v0.x, a0); a0 = fmaf(m0.y, v0.y, a0);
      a0 = fmaf(m0.z, v0.z, a0); a0 = fmaf(m0.w, v0.w, a0);
      a1 = fmaf(m1.x, v1.x, a1); a1 = fmaf(m1.y, v1.y, a1);
      a1 = fmaf(m1.z, v1.z, a1); a1 = fmaf(m1.w, v1.w, a1);
      a2 = fmaf(m2.x, v2.x, a2); a2 = fmaf(m2.y, v2.y, a2);
      a2 = fmaf(m2.z, v2.z, a2); a2 = fmaf(m2.w, v2.w, a2);
      a3 = fmaf(m3.x, v3.x, a3); a3 = fmaf(m3.y, v3.y, a3);
      a3 = fmaf(m3.z, v3.z, a3); a3 = fmaf(m3.w, v3.w, a3);
    }
    for (; c < end; c += L2C_WAVE) {
      const float4 m0 = NT ? ld4_stream(w4 + c) : w4[c];
      const float4 v0 = x4[c];
      a0 = fmaf(m0.x, v0.x, a0); a0 = fmaf(m0.y, v0.y, a0);
      a0 = fmaf(m0.z, v0.z, a0); a0 = fmaf(m0.w, v0.w, a0);
    }
  }
  const float acc = wave_sum((a0 + a1) + (a2 + a3));
  const int w = static_cast<int>(threadIdx.x) / L2C_WAVE;
  if (lane == 0) slots[w] = acc;
  __syncthreads();
  if (live && part == 0 && lane == 0) out[row] = acc + slots[w + 1];
}

// Two-pass versions for rows longer than the register-resident limit.
__device__ inline void rmsnorm_row_generic(float *out, const float *in, const float *weight,
                                           int size, float eps, float *slots) {
  float ss = 0.0f;
  for (int j = threadIdx.x; j < size; j += blockDim.x) ss = fmaf(in[j], in[j], ss);
  ss = block_sum(ss, slots);
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(size) + eps);
  for (int j = threadIdx.x; j < size; j += blockDim.x) out[j] = in[j] * scale * weight[j];
}

__device__ inline void softmax_row_generic(float *out, const float *logits, int size,
                                           float *slots) {
  float m = -FLT_MAX;
  for (int j = threadIdx.x; j < size; j += blockDim.x) m = fmaxf(m, logits[j]);
  m = block_max(m, slots);
  float s = 0.0f;
  for (int j = threadIdx.x; j < size; j += blockDim.x) s += expf(logits[j] - m);
  s = block_sum(s, slots + 16);
  const float inv = 1.0f / s;
  // Separate loops so the kernel is also correct in place (out == logits).
  for (int j = threadIdx.x; j < size; j += blockDim.x) out[j] = expf(logits[j] - m) * inv;
}

}  // namespace l2c
