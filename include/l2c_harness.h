/*
 * l2c_harness.h -- C ABI of libl2c_host.so, the llama2c harness as a library.
 *
 * The reference's process contract (llama2c/llama2c_cuda_graph.cu:195-258 for
 * argv, :508-517 for the key=value line, exit code 0/1) is exposed in-process
 * so a caller can run one harness invocation without spawning the
 * llama2c_hip executable.
 */
#ifndef L2C_HARNESS_H
#define L2C_HARNESS_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Runs one harness invocation with argv[0..argc) exactly as the llama2c_hip
 * command line would (argv[0] is the program name), writes the key=value
 * result line (without newline) into line[0..capacity), and returns the exit
 * code the executable would return (0 valid, 1 usage/runtime/validation
 * failure). Errors are printed to stderr. Replaces main() of
 * llama2c/llama2c_cuda_graph.cu:260-540.
 */
int l2c_harness_main(int argc, const char *const *argv, char *line, size_t capacity);

/*
 * Compares dumps with the rules of llama2c/compare_dumps.py:26-135;
 * paths[0] is the reference dump. Prints the report to stdout and returns
 * 0 when every other dump matches, 1 otherwise.
 */
int l2c_compare_dumps(int count, const char *const *paths);

#ifdef __cplusplus
}
#endif

#endif /* L2C_HARNESS_H */
