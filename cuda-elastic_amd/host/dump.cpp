// Dump writer/reader and the dump comparer.
//
// L2CDUMP1 is the layout of llama2c/llama2c_common.h:16-32 (little-endian, no
// padding). L2CDUMP2 carries batched products: the same 32-byte header, then
// int32 matmul code and int32 0, then normalized[B*S], softmax[B*S] (f32),
// product[B*R], tolerance[B*R] (f32) and reference[B*R] (f64). Unchecked
// product elements of a sampled check hold NaN tolerance and reference.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>

#include "l2c_host.h"

namespace l2c_host {

bool write_dump(const std::string &path, const Options &o, const Outputs &out,
                const ProductCheck &check) {
  std::FILE *file = std::fopen(path.c_str(), "wb");
  if (file == nullptr) {
    std::fprintf(stderr, "cannot open dump file %s\n", path.c_str());
    return false;
  }
  const bool batched = matmul_is_batched(o.matmul);
  const size_t n = static_cast<size_t>(o.batch) * o.size;
  const size_t p = batched ? static_cast<size_t>(o.batch) * o.rows : static_cast<size_t>(o.rows);
  const bool deterministic = o.inputs.mode == InputMode::kDeterministic;
  const int32_t header[4] = {o.batch, o.size, o.rows, static_cast<int32_t>(o.inputs.mode)};
  const uint64_t seed = deterministic ? 0 : o.inputs.seed;
  bool ok = std::fwrite(batched ? "L2CDUMP2" : "L2CDUMP1", 1, 8, file) == 8 &&
            std::fwrite(header, sizeof(header), 1, file) == 1 &&
            std::fwrite(&seed, sizeof(seed), 1, file) == 1;
  if (ok && batched) {
    const int32_t extra[2] = {static_cast<int32_t>(o.matmul), 0};
    ok = std::fwrite(extra, sizeof(extra), 1, file) == 1;
  }
  ok = ok && std::fwrite(out.normalized, sizeof(float), n, file) == n &&
       std::fwrite(out.softmax, sizeof(float), n, file) == n &&
       std::fwrite(out.product, sizeof(float), p, file) == p &&
       check.tolerance.size() == p && check.reference.size() == p &&
       std::fwrite(check.tolerance.data(), sizeof(float), p, file) == p &&
       std::fwrite(check.reference.data(), sizeof(double), p, file) == p;
  ok = std::fclose(file) == 0 && ok;
  if (!ok) std::fprintf(stderr, "failed to write dump file %s\n", path.c_str());
  return ok;
}

bool read_dump(const std::string &path, Dump *d, std::string *error) {
  std::FILE *file = std::fopen(path.c_str(), "rb");
  if (file == nullptr) {
    *error = path + ": cannot open";
    return false;
  }
  std::fseek(file, 0, SEEK_END);
  const long length = std::ftell(file);
  std::fseek(file, 0, SEEK_SET);
  std::vector<char> data(length > 0 ? static_cast<size_t>(length) : 0);
  const bool read_ok = length >= 0 && std::fread(data.data(), 1, data.size(), file) == data.size();
  std::fclose(file);
  if (!read_ok) {
    *error = path + ": read error";
    return false;
  }
  if (data.size() < 32 || (std::memcmp(data.data(), "L2CDUMP1", 8) != 0 &&
                           std::memcmp(data.data(), "L2CDUMP2", 8) != 0)) {
    *error = path + ": not a llama2c dump";
    return false;
  }
  d->magic.assign(data.data(), 8);
  int32_t header[4];
  std::memcpy(header, data.data() + 8, 16);
  std::memcpy(&d->seed, data.data() + 24, 8);
  d->batch = header[0];
  d->size = header[1];
  d->rows = header[2];
  d->inputs = header[3];
  size_t offset = 32;
  const bool v2 = d->magic == "L2CDUMP2";
  if (v2) {
    if (data.size() < 40) {
      *error = path + ": truncated in header";
      return false;
    }
    std::memcpy(&d->matmul, data.data() + 32, 4);
    offset = 40;
  }
  if (d->batch < 0 || d->size < 0 || d->rows < 0) {
    *error = path + ": bad header";
    return false;
  }
  const size_t n = static_cast<size_t>(d->batch) * d->size;
  const size_t p = v2 ? static_cast<size_t>(d->batch) * d->rows : static_cast<size_t>(d->rows);
  auto take = [&](const char *name, void *dst, size_t count, size_t width) {
    if (data.size() - offset < count * width) {
      *error = path + ": truncated in " + name;
      return false;
    }
    std::memcpy(dst, data.data() + offset, count * width);
    offset += count * width;
    return true;
  };
  d->normalized.resize(n);
  d->softmax.resize(n);
  d->product.resize(p);
  d->tolerance.resize(p);
  d->reference.resize(p);
  if (!take("normalized", d->normalized.data(), n, 4) || !take("softmax", d->softmax.data(), n, 4) ||
      !take("product", d->product.data(), p, 4) ||
      !take("product_tolerance", d->tolerance.data(), p, 4) ||
      !take("product_reference", d->reference.data(), p, 8))
    return false;
  if (offset != data.size()) {
    *error = path + ": " + std::to_string(data.size() - offset) + " trailing bytes";
    return false;
  }
  return true;
}

namespace {

struct Stat {
  double ratio = 0, abs = 0;
};

// max |a - b| / tol and max |a - b| over elements with a finite tolerance;
// any non-finite difference makes both infinite (llama2c/compare_dumps.py:78-82).
template <typename A, typename B, typename T>
Stat stat(size_t n, A a, B b, T tol) {
  Stat s;
  for (size_t i = 0; i < n; ++i) {
    const double t = tol(i);
    if (std::isnan(t)) continue;  // unchecked element of a sampled batched check
    const double diff = std::fabs(static_cast<double>(a(i)) - static_cast<double>(b(i)));
    if (!std::isfinite(diff)) return {std::numeric_limits<double>::infinity(),
                                      std::numeric_limits<double>::infinity()};
    s.abs = std::max(s.abs, diff);
    s.ratio = std::max(s.ratio, diff / t);
  }
  return s;
}

Stat product_error(const Dump &d) {
  return stat(d.product.size(), [&](size_t i) { return d.product[i]; },
              [&](size_t i) { return d.reference[i]; },
              [&](size_t i) { return static_cast<double>(d.tolerance[i]); });
}

const char *base_name(const std::string &path) {
  const size_t slash = path.find_last_of('/');
  return path.c_str() + (slash == std::string::npos ? 0 : slash + 1);
}

}  // namespace

bool compare_dumps(const std::vector<std::string> &paths) {
  if (paths.size() < 2) return false;
  Dump ref;
  std::string error;
  if (!read_dump(paths[0], &ref, &error)) {
    std::printf("%s\n", error.c_str());
    return false;
  }
  std::printf("  shape batch=%d size=%d rows=%d inputs=%d seed=%llu matmul=%d\n", ref.batch, ref.size,
              ref.rows, ref.inputs, static_cast<unsigned long long>(ref.seed), ref.matmul);
  Stat pe = product_error(ref);
  std::printf("  %s: reference; product error vs double reference %.3e (%.2e of tolerance)\n",
              base_name(paths[0]), pe.abs, pe.ratio);
  bool ok = true;
  for (size_t k = 1; k < paths.size(); ++k) {
    Dump other;
    if (!read_dump(paths[k], &other, &error)) {
      std::printf("  %s\n", error.c_str());
      ok = false;
      continue;
    }
    if (other.magic != ref.magic || other.batch != ref.batch || other.size != ref.size ||
        other.rows != ref.rows || other.inputs != ref.inputs || other.seed != ref.seed ||
        other.matmul != ref.matmul) {
      std::printf("  %s: header differs from the reference dump\n", base_name(paths[k]));
      ok = false;
      continue;
    }
    const size_t n = ref.normalized.size(), p = ref.product.size();
    const Stat sn = stat(n, [&](size_t i) { return other.normalized[i]; },
                         [&](size_t i) { return ref.normalized[i]; }, [](size_t) { return 3.0e-4; });
    const Stat ss = stat(n, [&](size_t i) { return other.softmax[i]; },
                         [&](size_t i) { return ref.softmax[i]; }, [&](size_t i) {
                           return 1.0e-9 + 1.0e-3 * std::fabs(static_cast<double>(ref.softmax[i]));
                         });
    const Stat sp = stat(p, [&](size_t i) { return other.product[i]; },
                         [&](size_t i) { return ref.product[i]; },
                         [&](size_t i) { return static_cast<double>(ref.tolerance[i]); });
    const Stat oe = product_error(other);
    const bool same = std::memcmp(other.normalized.data(), ref.normalized.data(), n * 4) == 0 &&
                      std::memcmp(other.softmax.data(), ref.softmax.data(), n * 4) == 0 &&
                      std::memcmp(other.product.data(), ref.product.data(), p * 4) == 0;
    const bool passed = sn.ratio <= 1.0 && ss.ratio <= 1.0 && sp.ratio <= 1.0 && oe.ratio <= 1.0;
    ok = ok && passed;
    std::printf("  %s: %s%s; normalized: max|diff|=%.3e (%.2e of tol) softmax: max|diff|=%.3e "
                "(%.2e of tol) product: max|diff|=%.3e (%.2e of tol); product error vs double "
                "reference %.3e (%.2e of tolerance)\n",
                base_name(paths[k]), passed ? "PASS" : "FAIL", same ? " (bitwise identical)" : "",
                sn.abs, sn.ratio, ss.abs, ss.ratio, sp.abs, sp.ratio, oe.abs, oe.ratio);
  }
  return ok;
}

}  // namespace l2c_host
