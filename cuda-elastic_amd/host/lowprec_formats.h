// Device encodings of the lowprec classifier cases. For each case: the device
// planes that one [rows][width] FP32 operand converts into, the launches that
// fill them, the classifier contraction over two encoded operands, and the
// host's reading of the planes' bytes back into one code per value, so the
// application can compare them bit for bit with the host quantizer
// (lowprec_reference.h). Formats, rounding and layouts: spec.json "formats",
// "rounding", "mxfp6", "nvfp4", "layout" of experiments/blackwell/lowprec; the
// device layouts are this build's own (include/l2c.h).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "decoder_contract.h"
#include "lowprec_reference.h"

namespace lowprec {

// One encoded operand on the device: its planes in the order its format lists
// them (codes, scales, ...), each a separate allocation.
struct DeviceTensor {
  long long rows = 0, width = 0;
  std::vector<l2c_decoder::DeviceArray<uint8_t>> planes;
  std::vector<size_t> sizes;
  uint8_t *plane(size_t i) const { return planes[i].get(); }
  size_t total_bytes() const;
};

// Host copies of a tensor's planes, same order.
using PlaneBytes = std::vector<std::vector<uint8_t>>;

class Format {
 public:
  virtual ~Format() = default;
  virtual int id() const = 0;
  // Byte sizes of the planes of a [rows][width] operand; none for FP32, which
  // the contraction reads as it is.
  virtual std::vector<size_t> plane_sizes(long long rows, long long width) const = 0;
  // x [rows][width] FP32 on the device into t. With alpha given (NVFP4
  // activations), also *alpha = d(x) * *partner_decode on the device.
  virtual void encode(const float *x, DeviceTensor &t, float *alpha, const float *partner_decode,
                      hipStream_t stream) = 0;
  // A device word (zero between steps) that the step's rmsnorm fills with the
  // maximum |x| of the activations it writes (l2c_decoder_rmsnorm_absmax), for
  // a format whose encoding needs the tensor maximum (NVFP4); else null.
  virtual unsigned *activation_absmax() { return nullptr; }
  // encode() for a step's activations, after the rmsnorm that filled
  // activation_absmax() when the format has one.
  virtual void encode_activations(const float *x, DeviceTensor &t, float *alpha, const float *partner_decode,
                                  hipStream_t stream) {
    encode(x, t, alpha, partner_decode, stream);
  }
  // Device address of a tensor's FP32 decode scale d (NVFP4), else null.
  virtual const float *decode_scale(const DeviceTensor &) const { return nullptr; }
  // logits[batch][vocab] = x . w^T over the encoded operands, times *alpha when
  // alpha is given; x32 / w32 are the FP32 operands (the FP32 control's).
  virtual void contract(float *logits, const float *x32, const DeviceTensor &x, const float *w32,
                        const DeviceTensor &w, const float *alpha, int batch, int width, int vocab,
                        hipStream_t stream) = 0;
  // The planes' bytes as one code per value and one scale byte per
  // [rows][width / block] block. A plane that disagrees with the codes (the
  // NVFP4 bf16 expansion) is described in *defect.
  virtual Quantized unpack(const PlaneBytes &planes, long long rows, long long width, std::string *defect) const = 0;

  DeviceTensor allocate(long long rows, long long width) const;
};

std::unique_ptr<Format> make_format(int lowprec_case);

PlaneBytes download(const DeviceTensor &t);
// Every plane filled with 0xFF bytes (stream-ordered).
void poison(const DeviceTensor &t, hipStream_t stream);

}  // namespace lowprec
