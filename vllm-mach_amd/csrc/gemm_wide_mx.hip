// The dense MX launches of the wide (prefill) GEMM, compiled as their own translation
// unit so that they take their own scheduling flags (build.py FILE_FLAGS): the
// iterative instruction-level-parallelism schedule measured 27.8 -> 27.0 us at c2's
// M = 512 and 34.9 -> 34.4 us at c4's M = 128, while it slowed the block-FP8 and grouped
// instantiations, which gemm_wide.hip keeps.
#define MXL_WIDE_MX_DENSE_ONLY 1
#include "gemm_wide.hip"
