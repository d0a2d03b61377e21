// l2c_compare: the dump comparer of the check flow, restating
// llama2c/compare_dumps.py (usage: l2c_compare REFERENCE.bin OTHER.bin ...).
// Exit 0 when every dump matches, 1 on a mismatch, 2 on a usage error.
#include <cstdio>
#include <string>
#include <vector>

#include "l2c_host.h"

int main(int argc, char **argv) {
  if (argc < 3) {
    std::fprintf(stderr, "Usage: %s REFERENCE.bin OTHER.bin [OTHER.bin ...]\n", argv[0]);
    return 2;
  }
  std::vector<std::string> paths(argv + 1, argv + argc);
  return l2c_host::compare_dumps(paths) ? 0 : 1;
}
