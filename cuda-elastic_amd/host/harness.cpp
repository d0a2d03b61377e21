// The whole command-line program as a function, so the same code runs as the
// llama2c_hip executable and in-process (l2c_harness_main) for a caller that
// loads libl2c_host.so.
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "../../include/l2c_harness.h"
#include "l2c_host.h"

namespace l2c_host {

int harness_main(int argc, const char *const *argv, std::string *line, bool print) {
  Options o;
  std::string error;
  if (!parse_options(argc, argv, &o, &error)) {
    if (!error.empty()) std::fprintf(stderr, "%s\n", error.c_str());
    else std::fputs(usage_text(argc > 0 ? argv[0] : "llama2c_hip").c_str(), stderr);
    return EXIT_FAILURE;
  }
  Inputs in;
  fill_inputs(o.inputs, o.batch, o.size, o.rows, &in);
  RunResult r;
  std::vector<float> normalized, softmax, product;
  QuantOperands q;
  if (!run(o, in, &r, &normalized, &softmax, &product, &q)) {
    std::fprintf(stderr, "%s\n", r.error.c_str());
    return EXIT_FAILURE;
  }
  const Outputs out{normalized.data(), softmax.data(), product.data()};
  Validation v = validate_all(o, in, out, matmul_is_quantized(o.matmul) ? &q : nullptr);
  if (!v.valid) std::fprintf(stderr, "Output validation failed\n");
  if (!o.inputs.dump_path.empty() && !write_dump(o.inputs.dump_path, o, out, v.product))
    v.valid = false;
  *line = result_line(o, r, v);
  if (print) {
    std::printf("%s\n", line->c_str());
    std::fflush(stdout);
  }
  return v.valid ? EXIT_SUCCESS : EXIT_FAILURE;
}

}  // namespace l2c_host

extern "C" int l2c_harness_main(int argc, const char *const *argv, char *line, size_t capacity) {
  std::string text;
  const int code = l2c_host::harness_main(argc, argv, &text, false);
  if (line != nullptr && capacity > 0) {
    std::strncpy(line, text.c_str(), capacity - 1);
    line[capacity - 1] = '\0';
  }
  return code;
}

extern "C" int l2c_compare_dumps(int count, const char *const *paths) {
  std::vector<std::string> list(paths, paths + count);
  return l2c_host::compare_dumps(list) ? 0 : 1;
}
