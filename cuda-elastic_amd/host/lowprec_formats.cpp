// The four classifier formats of the lowprec experiment as device encoders,
// contractions and host readers (lowprec_formats.h).
#include "lowprec_formats.h"

#include <cstring>
#include <numeric>

#include "../../include/l2c.h"
#include "app_protocol.h"
#include "parallel.h"

namespace lowprec {
namespace {

int host_threads() {
  return static_cast<int>(std::max(1u, std::min(16u, std::thread::hardware_concurrency())));
}

// Calls f(r) for every row, rows split over the host threads.
template <typename F>
void each_row(long long rows, F f) {
  l2c_host::parallel_ranges(static_cast<size_t>(rows), host_threads(), [&](size_t r0, size_t r1, size_t) {
    for (size_t r = r0; r < r1; ++r) f(static_cast<long long>(r));
  });
}

// Control: the FP32 operands go to the decoder's own FP32 classifier.
class Fp32 final : public Format {
 public:
  int id() const override { return kFp32; }
  std::vector<size_t> plane_sizes(long long, long long) const override { return {}; }
  void encode(const float *, DeviceTensor &, float *, const float *, hipStream_t) override {}
  void contract(float *logits, const float *x32, const DeviceTensor &, const float *w32, const DeviceTensor &,
                const float *, int batch, int width, int vocab, hipStream_t stream) override {
    APP_L2C(l2c_matmul(logits, x32, w32, batch, width, vocab, stream));
  }
  Quantized unpack(const PlaneBytes &, long long, long long, std::string *) const override { return {}; }
};

// One plane: the bf16 bits of every value.
class Bf16 final : public Format {
 public:
  int id() const override { return kBf16; }
  std::vector<size_t> plane_sizes(long long rows, long long width) const override {
    return {static_cast<size_t>(rows * width) * 2};
  }
  void encode(const float *x, DeviceTensor &t, float *, const float *, hipStream_t stream) override {
    APP_L2C(l2c_to_bf16_x4(reinterpret_cast<uint16_t *>(t.plane(0)), x, t.rows * t.width, stream));
  }
  void contract(float *logits, const float *, const DeviceTensor &x, const float *, const DeviceTensor &w,
                const float *, int batch, int width, int vocab, hipStream_t stream) override {
    APP_L2C(l2c_matmul_bf16(logits, reinterpret_cast<const uint16_t *>(x.plane(0)),
                            reinterpret_cast<const uint16_t *>(w.plane(0)), nullptr, batch, width, vocab, stream));
  }
  Quantized unpack(const PlaneBytes &planes, long long rows, long long width, std::string *) const override {
    Quantized q;
    q.codes.resize(static_cast<size_t>(rows * width));
    std::memcpy(q.codes.data(), planes[0].data(), q.codes.size() * 2);
    return q;
  }
};

// Planes: E3M2 codes and UE8M0 scales, both in the tiled operand layout of
// l2c_quantize_mxfp6 (rows padded to a multiple of 32; for each 128-value
// step t of the width, codes [t][row / 32][block b of 4][row % 32][24 bytes]
// and scales [t][row][b]).
class Mxfp6 final : public Format {
 public:
  int id() const override { return kMxfp6; }
  std::vector<size_t> plane_sizes(long long rows, long long width) const override {
    size_t codes = 0, scales = 0;
    APP_L2C(l2c_mxfp6_bytes(static_cast<int>(rows), static_cast<int>(width), &codes, &scales));
    return {codes, scales};
  }
  void encode(const float *x, DeviceTensor &t, float *, const float *, hipStream_t stream) override {
    APP_L2C(l2c_quantize_mxfp6(t.plane(0), t.plane(1), x, static_cast<int>(t.rows), static_cast<int>(t.width),
                               stream));
  }
  void contract(float *logits, const float *, const DeviceTensor &x, const float *, const DeviceTensor &w,
                const float *, int batch, int width, int vocab, hipStream_t stream) override {
    APP_L2C(l2c_matmul_mxfp6(logits, x.plane(0), x.plane(1), w.plane(0), w.plane(1), batch, width, vocab, stream));
  }
  Quantized unpack(const PlaneBytes &planes, long long rows, long long width, std::string *) const override {
    const long long padded = (rows + 31) / 32 * 32, blocks = width / 32;
    Quantized q;
    q.codes.resize(static_cast<size_t>(rows * width));
    q.scales.resize(static_cast<size_t>(rows * blocks));
    each_row(rows, [&](long long r) {
      for (long long kb = 0; kb < blocks; ++kb) {
        const long long step = kb / 4, lane = kb % 4;
        const size_t block_at = static_cast<size_t>((((step * (padded / 32) + r / 32) * 4 + lane) * 32 + r % 32) * 24);
        uint16_t *out = &q.codes[static_cast<size_t>(r * width + kb * 32)];
        for (long long j = 0; j < 32; ++j) out[j] = static_cast<uint16_t>(unpack_e3m2(&planes[0][block_at], j));
        q.scales[static_cast<size_t>(r * blocks + kb)] = planes[1][static_cast<size_t>((step * padded + r) * 4 + lane)];
      }
    });
    return q;
  }
};

// Planes: E2M1 codes (two per byte, row-major), UE4M3 scales [rows][width/16],
// the exact bf16 value of every element (what the contraction multiplies),
// and the tensor's FP32 encode and decode scales (s, d). Owns the partial
// maxima workspace of the tensor-scale reduction (weights), and the word the
// step's rmsnorm raises to the activations' maximum (the scales kernel clears
// it), so a step skips the separate maximum pass over its activations.
class Nvfp4 final : public Format {
 public:
  enum Plane { kCodes = 0, kScales = 1, kExpanded = 2, kTensor = 3 };
  // The maximum word is allocated and cleared here, at set-up, never while a
  // step may be under stream capture.
  Nvfp4() : absmax_(l2c_decoder::device_array<unsigned>(1)) {
    APP_HIP(hipMemset(absmax_.get(), 0, sizeof(unsigned)));
  }
  int id() const override { return kNvfp4; }
  std::vector<size_t> plane_sizes(long long rows, long long width) const override {
    const size_t n = static_cast<size_t>(rows * width);
    return {n / 2, n / 16, n * 2, 2 * sizeof(float)};
  }
  void encode(const float *x, DeviceTensor &t, float *alpha, const float *partner_decode, hipStream_t stream) override {
    if (!partials_) partials_ = l2c_decoder::device_array<float>(L2C_NVFP4_PARTIALS);
    float *tensor = reinterpret_cast<float *>(t.plane(kTensor));
    APP_L2C(l2c_nvfp4_tensor_scales(tensor, alpha, alpha ? partner_decode : nullptr, x, t.rows * t.width,
                                    partials_.get(), stream));
    APP_L2C(l2c_quantize_nvfp4(t.plane(kCodes), t.plane(kScales), reinterpret_cast<uint16_t *>(t.plane(kExpanded)), x,
                               tensor, static_cast<int>(t.rows), static_cast<int>(t.width), stream));
  }
  unsigned *activation_absmax() override { return absmax_.get(); }
  void encode_activations(const float *x, DeviceTensor &t, float *alpha, const float *partner_decode,
                          hipStream_t stream) override {
    float *tensor = reinterpret_cast<float *>(t.plane(kTensor));
    APP_L2C(l2c_nvfp4_tensor_scales_absmax(tensor, alpha, alpha ? partner_decode : nullptr, activation_absmax(),
                                           stream));
    APP_L2C(l2c_quantize_nvfp4(t.plane(kCodes), t.plane(kScales), reinterpret_cast<uint16_t *>(t.plane(kExpanded)), x,
                               tensor, static_cast<int>(t.rows), static_cast<int>(t.width), stream));
  }
  const float *decode_scale(const DeviceTensor &t) const override {
    return reinterpret_cast<const float *>(t.plane(kTensor)) + 1;
  }
  void contract(float *logits, const float *, const DeviceTensor &x, const float *, const DeviceTensor &w,
                const float *alpha, int batch, int width, int vocab, hipStream_t stream) override {
    APP_L2C(l2c_matmul_bf16(logits, reinterpret_cast<const uint16_t *>(x.plane(kExpanded)),
                            reinterpret_cast<const uint16_t *>(w.plane(kExpanded)), alpha, batch, width, vocab,
                            stream));
  }
  Quantized unpack(const PlaneBytes &planes, long long rows, long long width, std::string *defect) const override {
    Quantized q;
    q.codes.resize(static_cast<size_t>(rows * width));
    q.scales = planes[kScales];
    float tensor[2];
    std::memcpy(tensor, planes[kTensor].data(), sizeof tensor);
    q.decode = tensor[1];
    each_row(rows, [&](long long r) {
      const uint8_t *packed = &planes[kCodes][static_cast<size_t>(r * (width / 2))];
      for (long long k = 0; k < width; ++k) q.codes[static_cast<size_t>(r * width + k)] = static_cast<uint16_t>(unpack_e2m1(packed, k));
    });
    // Each bf16 the contraction multiplies must be its code's value times its
    // block scale's, exactly.
    const uint16_t *expanded = reinterpret_cast<const uint16_t *>(planes[kExpanded].data());
    std::vector<long long> off(static_cast<size_t>(rows), 0);
    each_row(rows, [&](long long r) {
      for (long long k = 0; k < width; ++k)
        off[static_cast<size_t>(r)] +=
            bf16_value(expanded[r * width + k]) != static_cast<double>(dequantized(kNvfp4, q, width, r, k));
    });
    const long long bad = std::accumulate(off.begin(), off.end(), 0LL);
    if (bad && defect) *defect = std::to_string(bad) + " bf16 expansion values differ from their codes";
    return q;
  }

 private:
  l2c_decoder::DeviceArray<float> partials_;
  l2c_decoder::DeviceArray<unsigned> absmax_;
};

}  // namespace

size_t DeviceTensor::total_bytes() const { return std::accumulate(sizes.begin(), sizes.end(), size_t{0}); }

DeviceTensor Format::allocate(long long rows, long long width) const {
  DeviceTensor t;
  t.rows = rows;
  t.width = width;
  t.sizes = plane_sizes(rows, width);
  for (size_t bytes : t.sizes) t.planes.push_back(l2c_decoder::device_array<uint8_t>(bytes));
  return t;
}

std::unique_ptr<Format> make_format(int lowprec_case) {
  switch (lowprec_case) {
    case kFp32: return std::make_unique<Fp32>();
    case kBf16: return std::make_unique<Bf16>();
    case kMxfp6: return std::make_unique<Mxfp6>();
    case kNvfp4: return std::make_unique<Nvfp4>();
    default: appproto::abort_run(appproto::kUsage, "unknown lowprec case %d", lowprec_case);
  }
}

PlaneBytes download(const DeviceTensor &t) {
  PlaneBytes out(t.planes.size());
  for (size_t i = 0; i < t.planes.size(); ++i) {
    out[i].resize(t.sizes[i]);
    APP_HIP(hipMemcpy(out[i].data(), t.plane(i), t.sizes[i], hipMemcpyDeviceToHost));
  }
  return out;
}

void poison(const DeviceTensor &t, hipStream_t stream) {
  for (size_t i = 0; i < t.planes.size(); ++i) APP_HIP(hipMemsetAsync(t.plane(i), 0xFF, t.sizes[i], stream));
}

}  // namespace lowprec
