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

/*
 * The llama2c decoder application (loom-private/llama2c-decoder) under the
 * loom_private protocol: argv as the llama2c_decoder_hip command line
 * (--preset, --launch direct|graph|both, --action check|bench|profile,
 * --iterations, --warmup, --set key=value, --asset, --json-out). Returns the
 * exit code the executable would return: 0 pass, 1 output mismatch, 2 usage
 * or invalid dimensions, 3 missing asset, 70 HIP error.
 *   l2c_decoder_main writes the one-line JSON result record into
 *     record[0..capacity) (empty if the run ended before it was built);
 *   l2c_decoder_run prints "RESULT <record>" to stdout instead.
 * Diagnostics go to stderr. Replaces main() of
 * applications/loom_private/decoder/decoder.cu:411-412 with
 * applications/loom_private/common/lp_harness.cuh:453-596.
 */
int l2c_decoder_main(int argc, const char *const *argv, char *record, size_t capacity);
int l2c_decoder_run(int argc, const char *const *argv);

/*
 * The lowprec classifier experiment (experiments/blackwell/lowprec): the
 * decoder above with only its classifier replaced. lowprec_case selects the
 * case the reference selects at compile time (decoder_lowprec.cu:1-35,
 * -DLP_LOWPREC_CASE): 0 fp32, 1 bf16, 2 mxfp6, 3 nvfp4. argv is the command
 * line of the reference's case binaries: the loom_private options of
 * l2c_decoder_main (with --set fixture=0..3), or --selftest (the device
 * quantizer against the host reference on crafted rows; exit 0 or 1), or
 * --accuracy [--json-out PATH] (spec.json "accuracy"). Replaces main() of
 * decoder_lowprec.cu:1414-1420.
 *   l2c_lowprec_main writes the JSON record into record[0..capacity);
 *   l2c_lowprec_run prints "RESULT <record>" to stdout instead.
 */
int l2c_lowprec_main(int lowprec_case, int argc, const char *const *argv, char *record, size_t capacity);
int l2c_lowprec_run(int lowprec_case, int argc, const char *const *argv);

/*
 * The application's host reference, for tests: l2c_lowprec_host_quantize
 * quantizes x [rows][width] as case lowprec_case (1..3) converts it, by table
 * search (codes unpacked one per value, bf16 bits for case 1; scales one per
 * block; *decode = the NVFP4 tensor decode scale); l2c_lowprec_fixture writes
 * the dense fixture of spec.json "fixtures"; l2c_lowprec_crafted the self-test
 * matrix. Return 0, or 2 for invalid arguments.
 */
int l2c_lowprec_host_quantize(int lowprec_case, const float *x, int rows, int width, unsigned short *codes,
                              unsigned char *scales, float *decode);
int l2c_lowprec_fixture(int seed, int width, int vocab, float *embedding, float *classifier);
int l2c_lowprec_crafted(int rows, int width, float *out);

#ifdef __cplusplus
}
#endif

#endif /* L2C_HARNESS_H */
