// One case of the lowprec classifier experiment (L2C_LOWPREC_CASE: 0 fp32,
// 1 bf16, 2 mxfp6, 3 nvfp4), as the reference builds one binary per case.
#include "../../include/l2c_harness.h"

#ifndef L2C_LOWPREC_CASE
#error "build with -DL2C_LOWPREC_CASE=0 (fp32), 1 (bf16), 2 (mxfp6) or 3 (nvfp4)"
#endif

int main(int argc, char **argv) { return l2c_lowprec_run(L2C_LOWPREC_CASE, argc, argv); }
