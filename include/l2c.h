/*
 * l2c.h -- C ABI of the MI355X (gfx950) llama2c hot path: rmsnorm, softmax and
 * the W.x matmul, as hand-written HIP kernels in libl2c.so.
 *
 * Every entry point only enqueues work on `stream`. It does not allocate,
 * synchronize or read device data on the host, so every call may be recorded
 * into a hipGraph with hipStreamBeginCapture. All pointers are caller-owned
 * device memory. float pointers must be 4-byte aligned; the kernels take
 * 16-byte vector paths when a row's address allows it and scalar paths
 * otherwise, so any alignment the HIP allocator hands out plus any row
 * offset is accepted.
 *
 * Return value: 0 (hipSuccess) or a hipError_t value. Bad arguments give
 * hipErrorInvalidValue (1) and enqueue nothing; a failed launch returns the
 * error reported by hipGetLastError after the launch, as the reference checks
 * cudaGetLastError after each launch (llama2c/llama2c_cuda_graph.cu:357,360,367).
 * l2c_strerror() names any returned code.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   l2c_rmsnorm   rmsnorm_kernel        llama2c/llama2c_cuda_graph.cu:58-78 (launch :355-357)
 *   l2c_softmax   softmax_kernel        llama2c/llama2c_cuda_graph.cu:82-115 (launch :358-360)
 *   l2c_matvec    matmul_kernel / matmul_coalesced_kernel
 *                                       llama2c/llama2c_cuda_graph.cu:119-162 (launch :361-367)
 *   l2c_fused     llama2c_sota_kernel   llama2c/llama2c_sota.cu:79-298 (launch :451-455)
 *   l2c_matmul    classifier_kernel     applications/loom_private/decoder/decoder.cu:79-125
 *   l2c_matmul_q  no kernel in the reference: the quantized-weight matmul of the
 *                 benchmark configuration (MXFP4 / per-row fp8 weights, bf16
 *                 activations); its codes follow experiments/blackwell/lowprec/reference.cpp:13-96
 *   l2c_matmul_qs the same product on the block-scaled matrix cores, activations
 *                 quantized to MXFP8: the analogue of the reference's block-scaled
 *                 CUTLASS GEMM, experiments/blackwell/lowprec/decoder_lowprec.cu:95-121
 *   l2c_decoder_init_model      init_model_kernel      applications/loom_private/decoder/decoder.cu:27-43
 *   l2c_decoder_rmsnorm         rmsnorm_kernel         applications/loom_private/decoder/decoder.cu:45-77
 *   l2c_decoder_softmax_argmax  softmax_argmax_kernel  applications/loom_private/decoder/decoder.cu:127-198
 *   (the decoder's classifier_kernel, decoder.cu:79-125, is l2c_matmul)
 */
#ifndef L2C_H
#define L2C_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Matrix-vector variants of l2c_matvec (the reference's `naive|coalesced` token). */
enum l2c_matvec_variant {
  L2C_MATVEC_NAIVE = 0,     /* one lane per output row (llama2c_cuda_graph.cu:119-128) */
  L2C_MATVEC_COALESCED = 1  /* rows streamed by whole wavefronts (llama2c_cuda_graph.cu:134-162) */
};

/* Weight formats of l2c_matmul_q. */
enum l2c_qformat {
  L2C_Q_MXFP4 = 0, /* e2m1 codes, two per byte (even k in the low nibble), one e8m0
                      scale byte per 32 consecutive k of a row: scales[r][k/32] */
  L2C_Q_FP8 = 1    /* e4m3 (OCP, bias 7, 0x7f/0xff NaN) codes, one byte each, and one
                      fp32 scale per row: scales[r] */
};

/*
 * out[b][j] = in[b][j] * (1 / sqrt(sum_j in[b][j]^2 / size + eps)) * weight[j]
 * for b < batch, j < size; rows are `size` floats apart.
 * Replaces rmsnorm_kernel, llama2c/llama2c_cuda_graph.cu:58-78.
 */
int l2c_rmsnorm(float *out, const float *in, const float *weight, int size, int batch,
                float eps, hipStream_t stream);

/*
 * out[b][j] = exp(logits[b][j] - max_b) / sum_j exp(logits[b][j] - max_b).
 * out may equal logits (in place).
 * Replaces softmax_kernel, llama2c/llama2c_cuda_graph.cu:82-115.
 */
int l2c_softmax(float *out, const float *logits, int size, int batch, hipStream_t stream);

/*
 * out[r] = sum_{c < cols} W[r][c] * x[c] for r < rows (W row-major, rows x cols).
 * variant: enum l2c_matvec_variant.
 * Replaces matmul_kernel / matmul_coalesced_kernel, llama2c/llama2c_cuda_graph.cu:119-162.
 */
int l2c_matvec(float *out, const float *x, const float *W, int cols, int rows, int variant,
               hipStream_t stream);

/*
 * All three operations of one llama2c iteration in one launch:
 *   normalized = rmsnorm(input, weight) over rms_rows rows,
 *   softmax    = softmax(logits) over softmax_rows rows,
 *   product    = matrix . input[0:size] over matmul_rows rows.
 * Any of the three row counts may be 0. Replaces llama2c_sota_kernel,
 * llama2c/llama2c_sota.cu:79-298 (its Work struct, :79-94).
 */
int l2c_fused(float *normalized, const float *input, const float *weight, float *softmax,
              const float *logits, float *product, const float *matrix, int size,
              int rms_rows, int softmax_rows, int matmul_rows, float eps, hipStream_t stream);

/*
 * Batched fp32 contraction on the fp32 matrix cores:
 *   out[b][r] = sum_{k < cols} W[r][k] * X[b][k], b < batch, r < rows
 * X is batch x cols, W is rows x cols, out is batch x rows, all row-major.
 * Same contraction as classifier_kernel,
 * applications/loom_private/decoder/decoder.cu:79-125 (logits = cls . norm).
 */
int l2c_matmul(float *out, const float *X, const float *W, int batch, int cols, int rows,
               hipStream_t stream);

/*
 * Quantized-weight contraction:
 *   out[b][r] = sum_k Xbf16[b][k] * dequant(Wq, scales)[r][k]
 * Xbf16: batch x cols bfloat16 (uint16 bit patterns); fmt: enum l2c_qformat.
 * Both formats need cols % 32 == 0 (l2c_quantize_fp8 itself takes any cols);
 * Xbf16 and Wq 16-byte aligned. cols % 64 == 0 runs the k-slice kernel
 * (MXFP4 scales at an even address), other shapes the first design.
 * No counterpart kernel in the reference (see the file header).
 */
int l2c_matmul_q(float *out, const void *Xbf16, const void *Wq, const void *scales, int fmt,
                 int batch, int cols, int rows, hipStream_t stream);

/*
 * Block-scaled quantized-weight contraction (the quantized-weight path on the
 * gfx950 scaled matrix cores, v_mfma_scale_f32_32x32x64_f8f6f4):
 *   out[b][r] = sum_k deq(MXFP8(Xbf16))[b][k] * deq(Wq, scales)[r][k]
 * Wq / scales / fmt are exactly l2c_matmul_q's weight operand. The activations
 * are first quantized on the device to MXFP8 into `workspace`: per 32
 * consecutive k one UE8M0 scale 2^X with X the smallest exponent for which
 * block max <= 448 * 2^X (ceil(log2(block max / 448)), clamped to
 * [-127, 127]; a zero block gets X = -127), elements e4m3(x * 2^-X)
 * nearest-even (the MX layout of experiments/blackwell/lowprec/spec.json
 * "mxfp6", with a scale that never clips the block maximum). The products of
 * the dequantized operands are exact; accumulation is FP32; the fp8 weights'
 * row scale multiplies each output.
 * Needs cols % 128 == 0; Xbf16, Wq and workspace 16-byte aligned, scales
 * 4-byte aligned; workspace_bytes >= l2c_mxfp8_workspace_bytes(batch, cols).
 *
 * Workspace layout (what l2c_quantize_mxfp8 writes): e4m3 codes row-major
 * [batch][cols] at offset 0; at offset round_up(batch * cols, 256) the scale
 * bytes in k-step tiles [cols / 128][Bp][4], Bp = batch rounded up to a
 * multiple of 4, byte j of a row's 4 = block j of that 128-k step, rows past
 * batch zero. l2c_mxfp8_workspace_bytes returns 0 for an unsupported shape.
 * Calls that share a workspace must be ordered on one stream.
 */
int l2c_matmul_qs(float *out, const void *Xbf16, const void *Wq, const void *scales, int fmt,
                  int batch, int cols, int rows, void *workspace, size_t workspace_bytes,
                  hipStream_t stream);
int l2c_quantize_mxfp8(void *workspace, size_t workspace_bytes, const uint16_t *Xbf16, int batch,
                       int cols, hipStream_t stream);
size_t l2c_mxfp8_workspace_bytes(int batch, int cols);

/*
 * l2c_matmul_qs without a workspace argument and without any allocation: the
 * MXFP8 activations go to a fixed scratch array inside the library
 * (L2C_QS_STATIC_SCRATCH_BYTES per GPU, held until the process ends; its
 * device address is looked up once per device on the first call there). No
 * counterpart in the reference: this entry point is for callers that cannot
 * allocate device memory (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Returns hipErrorInvalidValue when
 * l2c_mxfp8_workspace_bytes(batch, cols) exceeds the scratch size (batch *
 * cols up to about 24.4 million; the benchmark shape 1024 x 16384 needs
 * 16.5 MiB). Results equal l2c_matmul_qs's bit for bit. Every call on one GPU
 * uses that GPU's single scratch: calls that may overlap on one GPU (other
 * streams, other host threads) race and must be ordered by the caller.
 */
#define L2C_QS_STATIC_SCRATCH_BYTES (24u << 20)
int l2c_matmul_qs_static(float *out, const void *Xbf16, const void *Wq, const void *scales, int fmt,
                         int batch, int cols, int rows, hipStream_t stream);

/*
 * Quantizers for l2c_matmul_q's weight operand, run on the device (setup work,
 * outside any timed region):
 *   l2c_quantize_mxfp4: codes[r][k/2] (cols/2 bytes per row), scales[r][k/32];
 *     block scale exponent X = floor(log2(amax / 6)) clamped to [-127, 127]
 *     (amax = 0 gives X = -127 and zero codes); code = e2m1(w * 2^-X), nearest,
 *     ties to the even code, saturating at 6, -0 encoded as +0.
 *   l2c_quantize_fp8: codes[r][k], scales[r] = amax_r / 448 (1 if amax_r = 0);
 *     code = e4m3(w / scales[r]), nearest-even, saturating at 448.
 *   l2c_to_bf16: bf16 round-to-nearest-even of n floats.
 */
int l2c_quantize_mxfp4(uint8_t *codes, uint8_t *scales, const float *W, int rows, int cols,
                       hipStream_t stream);
int l2c_quantize_fp8(uint8_t *codes, float *scales, const float *W, int rows, int cols,
                     hipStream_t stream);
int l2c_to_bf16(uint16_t *out, const float *in, size_t n, hipStream_t stream);

/*
 * Low-precision classifier formats (experiments/blackwell/lowprec/spec.json
 * "formats", "rounding", "mxfp6", "nvfp4"; the reference's device quantizers
 * are decoder_lowprec.cu:202-340 and its GEMMs CUTLASS calls at
 * decoder_lowprec.cu:751-764). Every encoder rounds to nearest with ties to
 * the even code, saturates, and writes +0 for magnitudes that round to zero.
 *
 * l2c_quantize_mxfp6: x [rows][width] (width % 128 == 0, x 16-byte aligned) to
 *   E3M2 codes and one UE8M0 scale byte per 32 values: X = floor(log2(block
 *   max)) - 4 clamped to [-127, 127], scale code X + 127, elements E3M2(v * 2^-X);
 *   a zero block has scale 0 and codes 0. Output in the tiled operand layout of
 *   l2c_matmul_mxfp6, rows padded to Rp = 32 * ceil(rows / 32) (padding rows
 *   zero): codes [width/128][Rp/32][4][32][24 B], where 24 B are one 32-value
 *   block's codes as a little-endian 6-bit stream (value i at bits 6i..6i+5);
 *   scales [width/128][Rp][4 B], byte b for block b of each 128-value step.
 *   l2c_mxfp6_bytes gives both sizes. (The reference keeps rows contiguous and
 *   its scale bytes in CUTLASS's tile layout; the byte values are the same.)
 * l2c_nvfp4_tensor_scales: tensor_scales[0] = s = 2688 / max|x| (1 when the
 *   maximum is 0), tensor_scales[1] = d = 1 / s, and, when alpha is not NULL,
 *   *alpha = d * *other_decode, all FP32 on the device. partials: a device
 *   workspace of L2C_NVFP4_PARTIALS floats. Two launches, no atomics, no memset.
 * l2c_nvfp4_tensor_scales_absmax: the same three values from a maximum that
 *   l2c_decoder_rmsnorm_absmax left in *absmax_bits (the float's bits), which it
 *   then sets to 0 for the next one: one single-lane launch. No counterpart in
 *   the reference, whose tensor maximum is a separate pass over x; this pair
 *   saves the lowprec NVFP4 step that pass.
 * l2c_quantize_nvfp4: x [rows][width] (width % 16 == 0) to E2M1 codes (two per
 *   byte, even index in the low nibble) and UE4M3 scales[rows][width / 16]:
 *   scale code UE4M3((block max / 6) * s), codes E2M1((v * s) / f), f the scale's
 *   value, FP32 operations in this order; a zero scale code zeroes the block.
 *   s is read from tensor_scales[0] on the device. expanded_bf16 (optional,
 *   [rows][width]) receives each element's exact value code * f as bf16.
 *   x and expanded_bf16 16-byte aligned, codes 8-byte aligned.
 * l2c_to_bf16_x4: l2c_to_bf16 for n % 4 == 0 and 16-byte aligned input.
 */
#define L2C_NVFP4_PARTIALS 1024
int l2c_quantize_mxfp6(uint8_t *codes, uint8_t *scales, const float *x, int rows, int width,
                       hipStream_t stream);
int l2c_mxfp6_bytes(int rows, int width, size_t *code_bytes, size_t *scale_bytes);
int l2c_nvfp4_tensor_scales(float *tensor_scales, float *alpha, const float *other_decode,
                            const float *x, long long n, float *partials, hipStream_t stream);
int l2c_nvfp4_tensor_scales_absmax(float *tensor_scales, float *alpha, const float *other_decode,
                                   unsigned *absmax_bits, hipStream_t stream);
int l2c_quantize_nvfp4(uint8_t *codes, uint8_t *scales, uint16_t *expanded_bf16, const float *x,
                       const float *tensor_scales, int rows, int width, hipStream_t stream);
int l2c_to_bf16_x4(uint16_t *out, const float *in, long long n, hipStream_t stream);

/*
 * Classifier contractions of the lowprec cases, out[b][r] = sum_k X[b][k] W[r][k]
 * (X batch x cols, W rows x cols, out batch x rows, FP32 accumulation):
 * l2c_matmul_bf16: bf16 X and W on the bf16 matrix cores (cols % 32 == 0); every
 *   output is multiplied by *alpha when alpha (a device pointer) is not NULL.
 *   The bf16 case (CUTLASS Sm80 GEMM, decoder_lowprec.cu:82-89) and, on the exact
 *   bf16 expansions of NVFP4 operands with alpha = d_X * d_W, the NVFP4 case.
 * l2c_matmul_mxfp6: MXFP6 X and W in the tiled layout l2c_quantize_mxfp6 writes,
 *   on the scaled matrix cores (cols % 128 == 0, all four pointers 16-byte
 *   aligned). The MXFP6 case (CUTLASS SM120 block-scaled GEMM,
 *   decoder_lowprec.cu:90-121).
 */
int l2c_matmul_bf16(float *out, const uint16_t *X, const uint16_t *W, const float *alpha, int batch,
                    int cols, int rows, hipStream_t stream);
int l2c_matmul_mxfp6(float *out, const uint8_t *X, const uint8_t *Xscales, const uint8_t *W,
                     const uint8_t *Wscales, int batch, int cols, int rows, hipStream_t stream);

/*
 * Batched greedy decoder (applications/loom_private/decoder): one step is
 *   l2c_decoder_rmsnorm -> l2c_matmul(logits, normalized, classifier) ->
 *   l2c_decoder_softmax_argmax
 * over `batch` independent sequences whose current tokens live on the device.
 *
 * l2c_decoder_init_model: the synthetic model of the decoder's contract, on the
 *   device: embedding[t][j] = (j == t ? 4 : 1), classifier[r][j] =
 *   (j == (r + vocab - 1) % vocab ? 1 : 0) (both vocab x width), norm_weight = 1.
 * l2c_decoder_rmsnorm: normalized[b][j] = weight[j] * (scale_b * E[t_b][j]) with
 *   t_b = tokens[b], scale_b = 1 / sqrtf(sum_j E[t_b][j]^2 / width + 1e-5f); a token
 *   outside [0, vocab) gives a NaN row.
 * l2c_decoder_rmsnorm_absmax: the same, and the maximum of |normalized| over
 *   the batch (NaNs ignored) raised into *absmax_bits as a float's bits by
 *   atomic maximum (exact in any order); the word must start at 0 (or at a
 *   maximum to extend). No counterpart in the reference: it feeds
 *   l2c_nvfp4_tensor_scales_absmax.
 * l2c_decoder_softmax_argmax: probabilities[b][r] = expf(logits[b][r] - max_b) / sum_b;
 *   t = index of the first maximum probability (-1 if none); tokens[b] = t and
 *   generated[b * steps + step] = t.
 * Reductions run in a fixed order: results are deterministic.
 */
int l2c_decoder_init_model(float *embedding, float *classifier, float *norm_weight, int width,
                           int vocab, hipStream_t stream);
int l2c_decoder_rmsnorm(float *normalized, const int *tokens, const float *embedding,
                        const float *weight, int width, int vocab, int batch, hipStream_t stream);
int l2c_decoder_rmsnorm_absmax(float *normalized, const int *tokens, const float *embedding,
                               const float *weight, int width, int vocab, int batch,
                               unsigned *absmax_bits, hipStream_t stream);
int l2c_decoder_softmax_argmax(float *probabilities, const float *logits, int *tokens,
                               int *generated, int vocab, int batch, int steps, int step,
                               hipStream_t stream);

/*
 * bytes from device memory `src` to pinned host memory `host_dst`
 * (hipHostMalloc; on ROCm its host address is also its device address),
 * copied by a kernel that stores straight into host memory: the copy is a
 * kernel node when captured into a hipGraph, not a memcpy node. No
 * counterpart kernel in the reference, whose copy mode downloads with
 * cudaMemcpyAsync (llama2c/llama2c_cuda_graph.cu:369-374); the harness's
 * `hostwrite` token uses it in that place. 16-byte stores when both pointers
 * are 16-byte aligned, byte stores for the rest.
 */
int l2c_copy_to_host(void *host_dst, const void *src, size_t bytes, hipStream_t stream);

/* Operations named by l2c_launch_shape. */
enum l2c_op {
  L2C_OP_RMSNORM = 0,
  L2C_OP_SOFTMAX = 1,
  L2C_OP_MATVEC = 2,
  L2C_OP_FUSED = 3,
  L2C_OP_MATMUL = 4,
  L2C_OP_MATMUL_Q = 5,
  L2C_OP_MATMUL_QS = 6  /* the contraction kernel of l2c_matmul_qs */
};

/*
 * Launch shape the library uses for one call of `op` (batch vectors of `cols`
 * floats; `rows` matrix rows; variant = matvec variant or quantized format),
 * and how many of its workgroups fit on one CU at once, for the harness's
 * waves = grid / (blocks_per_cu * CUs) figures. The reference computes them
 * inline with cudaOccupancyMaxActiveBlocksPerMultiprocessor,
 * llama2c/llama2c_cuda_graph.cu:318-336. For L2C_OP_FUSED, batch is both the
 * rmsnorm and softmax row count.
 */
int l2c_launch_shape(int op, int batch, int cols, int rows, int variant, int *grid, int *block,
                     int *blocks_per_cu);

/* Name of a code returned by any l2c_* call. */
const char *l2c_strerror(int code);

/* Library version string; also proves the library loaded. */
const char *l2c_version(void);

#ifdef __cplusplus
}
#endif

#endif /* L2C_H */
