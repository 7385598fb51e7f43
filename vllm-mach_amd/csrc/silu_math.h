// exp() and the SwiGLU activation as fixed binary32 operation sequences, shared by the
// device code (mx_common.h) and the host generator of the activation table
// (silu_table_gen.cpp), so that both evaluate the same operations.  Compiled without
// contraction (-ffp-contract=off); fused steps call __builtin_fmaf explicitly.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MXL_HD __host__ __device__ __forceinline__
#else
#define MXL_HD static inline
#endif

namespace mxl {

// exp() with a fixed binary32 operation sequence: Cody-Waite reduction by ln2
// and the Cephes expf minimax polynomial (S. L. Moshier), explicit FMAs.
MXL_HD float mx_exp(float x) {
  // branch-free: the range limits select the result; the exponent is clamped before
  // the integer conversion so that it is defined for every x (NaN included)
  const float n = __builtin_rintf(x * 1.44269504088896341f);
  float r = __builtin_fmaf(n, -0.693359375f, x);
  r = __builtin_fmaf(n, 2.12194440e-4f, r);
  float p = 1.9875691500e-4f;
  p = __builtin_fmaf(p, r, 1.3981999507e-3f);
  p = __builtin_fmaf(p, r, 8.3334519073e-3f);
  p = __builtin_fmaf(p, r, 4.1665795894e-2f);
  p = __builtin_fmaf(p, r, 1.6666665459e-1f);
  p = __builtin_fmaf(p, r, 5.0000001201e-1f);
  const float r2 = r * r;
  const float y = __builtin_fmaf(p, r2, r) + 1.0f;
  const float nc = __builtin_fminf(__builtin_fmaxf(n, -300.0f), 300.0f);
  float e = __builtin_ldexpf(y, (int)nc);
  e = x < -87.0f ? 0.0f : e;
  return x > 88.0f ? __builtin_inff() : e;
}

// SiLU in binary32: g / (1 + exp(-g)) (mxfp8_mlp.py:96, swiglu_quant.py:56)
MXL_HD float mx_silu(float g) { return g / (1.0f + mx_exp(-g)); }

// The rounded activation bf16(silu(g)) of rules 0 and 1 is a function of the bf16 gate
// alone.  The table (kSiluAct, written at build time by silu_table_gen.cpp) holds it for
// the gate exponent fields kSiluELo .. kSiluEHi, 2^-24 <= |g| < 256, positive gates then
// negative ones: index (bits & 0x7FFF) - (kSiluELo << 7), plus kSiluSpan for a negative
// gate.  Gates outside it (zeros, tiny, huge, inf, NaN) take the arithmetic.
constexpr uint32_t kSiluELo = 103;
constexpr uint32_t kSiluEHi = 134;
constexpr uint32_t kSiluSpan = (kSiluEHi - kSiluELo + 1) << 7;
constexpr uint32_t kSiluEntries = 2 * kSiluSpan;

}  // namespace mxl
