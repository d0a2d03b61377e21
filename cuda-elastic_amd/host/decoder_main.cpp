// llama2c_decoder_hip: the loom-private/llama2c-decoder application as a
// command line (the program of applications/loom_private/decoder/decoder.cu).
#include "../../include/l2c_harness.h"

int main(int argc, char **argv) { return l2c_decoder_run(argc, argv); }
