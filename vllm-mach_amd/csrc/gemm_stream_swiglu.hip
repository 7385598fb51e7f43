// The one-row SwiGLU -> MX GEMM launch (gemm_stream_kernel with ROWP = rule: every
// wavefront computes its super-tiles' SiLU and MXFP8 codes of the row), compiled as its
// own translation unit so that it takes its own scheduling flags (build.py FILE_FLAGS):
// the instruction-level-parallelism schedule measured 9.38 against 9.90 us at c2's
// shape, while it slowed the other stream kernels.
#define MXL_STREAM_SWIGLU_ONLY 1
#include "gemm_stream.hip"
