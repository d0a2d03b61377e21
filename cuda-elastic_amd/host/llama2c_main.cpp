// llama2c_hip: the drop-in for the reference's llama2c_cuda_graph and
// llama2c_sota executables (same command line, key=value line, exit codes).
#include <string>

#include "l2c_host.h"

int main(int argc, char **argv) {
  std::string line;
  return l2c_host::harness_main(argc, argv, &line, true);
}
