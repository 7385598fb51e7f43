/*
 * CPU oracle for the quantized-linear hot path.  TEST INFRASTRUCTURE ONLY:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker.  The product path never calls it.
 *
 * Each function restates one algorithm of the reference (troycheng/vllm-mach
 * v0.4.0) in plain C with IEEE-754 binary32 arithmetic, round-to-nearest-even,
 * no FMA contraction (built with -ffp-contract=off; fused steps call fmaf
 * explicitly).  Citations are file:line in the reference tree.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ bits */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float mxo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* torch/c10 BFloat16 conversion: round-to-nearest-even, NaN -> 0x7FC0. */
uint16_t mxo_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
  uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7FFFu + lsb) >> 16);
}

static inline float bf16_round(float f) { return mxo_bf16_to_f32(mxo_f32_to_bf16(f)); }

/* -------------------------------------------------------------- E4M3 codec
 * E4M3 "fn": bias 7, 3 mantissa bits, no infinities, 0x7F/0xFF = NaN, max
 * finite 448.  Conversion follows torch's float -> float8_e4m3fn cast, which
 * is what the reference quantizer uses (mxfp8/reconstruct_model.py:48):
 * round-to-nearest-even onto the E4M3 grid, where a magnitude that rounds
 * past 448 (or is >= 480, or NaN) produces the NaN code.  No saturation.   */
uint8_t mxo_f32_to_e4m3(float f) {
  uint32_t u = f2u(f);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  uint32_t a = u & 0x7FFFFFFFu;
  if (a >= 0x43F00000u) return (uint8_t)(sign | 0x7F);   /* >= 480 or NaN */
  if (a < 0x3C800000u) {                                  /* < 2^-6: subnormal grid, step 2^-9 */
    float q = rintf(u2f(a) * 512.0f);                     /* exact scale, RNE to integer 0..8 */
    return (uint8_t)(sign | (uint8_t)q);
  }
  uint32_t odd = (a >> 20) & 1u;
  uint32_t r = (a - (120u << 23) + 0x7FFFFu + odd) >> 20; /* rebias 127->7, RNE to 3 bits */
  return (uint8_t)(sign | (uint8_t)r);                    /* 464 < |f| < 480 lands on 0x7F */
}

float mxo_e4m3_to_f32(uint8_t c) {
  uint32_t e = (c >> 3) & 0xF, m = c & 7;
  float s = (c & 0x80) ? -1.0f : 1.0f;
  if (e == 0xF && m == 7) return NAN;
  if (e == 0) return s * ldexpf((float)m, -9);
  return s * ldexpf((float)(8 + m), (int)e - 10);
}

/* --------------------------------------------------------------- FP6 codec
 * OCP MX v1.0 element formats (no Inf/NaN; conversion saturates to max
 * normal, round-to-nearest-even):  fmt 2 = E2M3 (bias 1, max 7.5),
 * fmt 3 = E3M2 (bias 3, max 28).  Code bit 5 is the sign.                 */
uint8_t mxo_f32_to_fp6(float f, int fmt) {
  uint32_t u = f2u(f);
  uint8_t sign = (uint8_t)((u >> 26) & 0x20u);
  uint32_t a = u & 0x7FFFFFFFu;
  int mbits = fmt == 2 ? 3 : 2, bias = fmt == 2 ? 1 : 3;
  uint32_t min_normal = (uint32_t)(127 + 1 - bias) << 23;
  uint32_t code;
  if (a > 0x7F800000u) return sign;                       /* NaN: not produced by the quantizer */
  if (a < min_normal) {                                   /* subnormal grid, step 2^(1-bias-mbits) */
    code = (uint32_t)rintf(ldexpf(u2f(a), bias - 1 + mbits));
  } else {
    int sh = 23 - mbits;
    uint32_t odd = (a >> sh) & 1u;
    uint64_t t = (uint64_t)a - ((uint64_t)(127 - bias) << 23) + ((1u << (sh - 1)) - 1) + odd;
    code = (uint32_t)(t >> sh);
  }
  if (code > 31) code = 31;                               /* saturate */
  return (uint8_t)(sign | code);
}

float mxo_fp6_to_f32(uint8_t c, int fmt) {
  int mbits = fmt == 2 ? 3 : 2, bias = fmt == 2 ? 1 : 3;
  uint32_t e = (c & 0x1F) >> mbits, m = c & ((1u << mbits) - 1);
  float s = (c & 0x20) ? -1.0f : 1.0f;
  if (e == 0) return s * ldexpf((float)m, 1 - bias - mbits);
  return s * ldexpf((float)((1u << mbits) + m), (int)e - bias - mbits);
}

/* FP6 packing: four 6-bit codes per three bytes, little-endian bit stream:
 * bits [6i, 6i+6) of the 24-bit group hold value i.  A 32-value MX block is
 * therefore 24 contiguous bytes.  (The reference fixes only the 4-in-3 shape,
 * mxfp6/dense.py:61-80; the bit order is this build's definition.)           */
void mxo_pack_fp6(const uint8_t* codes, int64_t n, uint8_t* out) {
  for (int64_t g = 0; g < n / 4; ++g) {
    uint32_t w = (uint32_t)(codes[4 * g] & 63) | ((uint32_t)(codes[4 * g + 1] & 63) << 6) |
                 ((uint32_t)(codes[4 * g + 2] & 63) << 12) | ((uint32_t)(codes[4 * g + 3] & 63) << 18);
    out[3 * g] = (uint8_t)w; out[3 * g + 1] = (uint8_t)(w >> 8); out[3 * g + 2] = (uint8_t)(w >> 16);
  }
}

void mxo_unpack_fp6(const uint8_t* packed, int64_t n, uint8_t* codes) {
  for (int64_t g = 0; g < n / 4; ++g) {
    uint32_t w = packed[3 * g] | ((uint32_t)packed[3 * g + 1] << 8) | ((uint32_t)packed[3 * g + 2] << 16);
    for (int i = 0; i < 4; ++i) codes[4 * g + i] = (uint8_t)((w >> (6 * i)) & 63);
  }
}

/* ------------------------------------------------------ MXFP8 scale rules */

/* Rule "floor_carry175": mxfp8/reconstruct_model.py:44-48 (quantize_block).
 * rounded = (bits(amax_bf16) + 32) & 0xFF80 keeps sign+exponent after a carry
 * that fires when the 7-bit mantissa is >= 96 (amax mantissa >= 1.75);
 * s = 127 + log2(rounded) - 8 = E(rounded) - 8, cast to uint8.  rounded == 0
 * (amax 0 or a small subnormal) gives log2 = -inf -> 0, matching the stored
 * known answer.  E(rounded) in 1..7 gives a negative float that torch's CPU
 * uint8 cast wraps modulo 256; that branch is unreachable at the configured
 * data and is not pinned by any reference vector.                           */
static uint8_t scale_floor_carry175(uint16_t amax_bf16) {
  uint32_t rounded = ((uint32_t)amax_bf16 + 32u) & 0xFF80u;
  uint32_t e = (rounded >> 7) & 0xFF;
  if (e == 0) return 0;
  return (uint8_t)((int)e - 8);
}

/* Rule "ceil_div448": mxfp6/mxfp8_mlp.py:100-105.  raw = max(amax/448, 1e-30)
 * (IEEE division), round the binary32 up to a power of two by adding
 * 0x7FFFFF and masking the exponent; the exponent field is the E8M0 code and
 * the element divisor is that power of two.                                 */
static uint32_t pow2_ceil_div448(float amax) {
  float raw = amax / 448.0f;
  if (!(raw >= 1.0e-30f)) raw = 1.0e-30f;
  return (f2u(raw) + 0x007FFFFFu) & 0x7F800000u;
}

/* Rule "rp_ue8m0": the FlashInfer mxfp8_quantize convention that the reference's
 * champion producer writes out (mxfp8/swiglu_quant.py:58-66).  raw = amax * r448
 * with r448 the reciprocal of 448; s = raw rounded toward +inf onto E8M0
 * (2^(s-127), s in 0..254, saturating at 254; raw <= 2^-127 gives 0);
 * inverse = 2^(127-s), 0 for s = 0 (the reference's where(scale > 0)) and for
 * s = 254 (2^-127 is subnormal and the reference's reciprocal flushes it);
 * codes = E4M3(min(max(v * inverse, -448), 448)), the clamp taken in that order
 * (a NaN product gives -448).  The reference takes rcp.approx.ftz of 448 on
 * NVIDIA hardware; this build uses the correctly rounded 1/448 (0x3B124925):
 * parity unpinned for that constant, whose exact value decides the scale only
 * where amax * r448 lands within an ulp of a power of two.                    */
static const float kRcp448 = 1.0f / 448.0f;

static uint8_t e8m0_rp(float raw) {
  uint32_t u = f2u(raw);
  if (u >= 0x7F800000u) return 254;          /* +inf (raw is never negative or NaN) */
  uint32_t e = u >> 23, m = u & 0x7FFFFFu;
  if (e == 0) return u <= 0x00400000u ? 0 : 1;  /* 2^-127 is the subnormal 0x00400000 */
  uint32_t s = e + (m != 0);
  return (uint8_t)(s > 254 ? 254 : s);
}

/* Quantize one 32-element block of binary32 values that are exactly bf16
 * (all values are bf16-representable).  rule 0 = floor_carry175, 1 = ceil_div448,
 * 2 = rp_ue8m0. */
static void quant_block32(const float* v, int rule, uint8_t* codes, uint8_t* scale) {
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) { float a = fabsf(v[i]); if (a > amax) amax = a; }
  if (rule == 2) {
    uint8_t s = e8m0_rp(amax * kRcp448);
    float inverse = (s == 0 || s == 254) ? 0.0f : ldexpf(1.0f, 127 - (int)s);
    for (int i = 0; i < 32; ++i) codes[i] = mxo_f32_to_e4m3(fminf(fmaxf(v[i] * inverse, -448.0f), 448.0f));
    *scale = s;
    return;
  }
  if (rule == 0) {
    uint8_t s = scale_floor_carry175(mxo_f32_to_bf16(amax));
    /* x / 2^(s-127) (reconstruct_model.py:47-48); an exact power-of-two divide */
    float div = ldexpf(1.0f, (int)s - 127);
    for (int i = 0; i < 32; ++i) codes[i] = mxo_f32_to_e4m3(v[i] / div);
    *scale = s;
  } else {
    uint32_t bits = pow2_ceil_div448(amax);
    float inverse = 1.0f / u2f(bits);                     /* mxfp8_mlp.py:104 */
    for (int i = 0; i < 32; ++i) codes[i] = mxo_f32_to_e4m3(v[i] * inverse);
    *scale = (uint8_t)(bits >> 23);
  }
}

/* Dynamic MXFP8 quantization of a bf16 matrix [rows, K] (K % 32 == 0) into
 * E4M3 codes [rows, K] and logical E8M0 scales [rows, K/32], both row-major.
 * rule 0 restates quantize_block (reconstruct_model.py:34-50).             */
void mxo_quant_mxfp8(const uint16_t* x, int64_t rows, int64_t K, int rule,
                     uint8_t* codes, uint8_t* scales) {
  float v[32];
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t b = 0; b < K / 32; ++b) {
      for (int i = 0; i < 32; ++i) v[i] = mxo_bf16_to_f32(x[r * K + b * 32 + i]);
      quant_block32(v, rule, codes + r * K + b * 32, scales + r * (K / 32) + b);
    }
}

/* ----------------------------------------------------------- SiLU / exp
 * exp() is specified here, not taken from a libm, so that the HIP producer
 * and this oracle evaluate the same binary32 operation sequence: Cody-Waite
 * reduction by ln2 (hi/lo split) and the Cephes expf minimax polynomial
 * (S. L. Moshier, Cephes Math Library), evaluated with explicit fmaf.
 * Inputs below -87 return 0 and above 88 return +inf; SiLU only uses
 * 1 + exp(-g), which rounds identically for any value under 2^-25.          */
/* Two-limb ("dual") MXFP8 activations, the contract of the reference's dual
 * path (src/vllm_mach/mxfp8/dual.py:45-50; docs/mxfp8-champion.md:12 "high plus
 * BF16-rounded residual, separate FP32 accumulators and final BF16 rounding").
 * The quantizer itself is in the absent mxfp6 wheel; this build defines it per
 * 32-block as: hi = MXFP8(x) under `rule`; residual r = bf16(x - deq(hi)) with
 * deq(hi) = E4M3(code) * 2^(s - 127) exact in binary32 and one f32 subtraction;
 * res = MXFP8(r) under the same rule.                                          */
void mxo_quant_mxfp8_dual(const uint16_t* x, int64_t rows, int64_t K, int rule, uint8_t* hi, uint8_t* s_hi,
                          uint8_t* res, uint8_t* s_res) {
  float v[32], rv[32];
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t b = 0; b < K / 32; ++b) {
      for (int i = 0; i < 32; ++i) v[i] = mxo_bf16_to_f32(x[r * K + b * 32 + i]);
      uint8_t* hc = hi + r * K + b * 32;
      uint8_t* hs = s_hi + r * (K / 32) + b;
      quant_block32(v, rule, hc, hs);
      for (int i = 0; i < 32; ++i) rv[i] = bf16_round(v[i] - ldexpf(mxo_e4m3_to_f32(hc[i]), (int)*hs - 127));
      quant_block32(rv, rule, res + r * K + b * 32, s_res + r * (K / 32) + b);
    }
}

float mxo_exp(float x) {
  if (x < -87.0f) return 0.0f;
  if (x > 88.0f) return INFINITY;
  float n = rintf(x * 1.44269504088896341f);
  float r = fmaf(n, -0.693359375f, x);
  r = fmaf(n, 2.12194440e-4f, r);
  float p = 1.9875691500e-4f;
  p = fmaf(p, r, 1.3981999507e-3f);
  p = fmaf(p, r, 8.3334519073e-3f);
  p = fmaf(p, r, 4.1665795894e-2f);
  p = fmaf(p, r, 1.6666665459e-1f);
  p = fmaf(p, r, 5.0000001201e-1f);
  float r2 = r * r;
  float y = fmaf(p, r2, r) + 1.0f;
  return ldexpf(y, (int)n);
}

/* SwiGLU -> MXFP8, mxfp6/mxfp8_mlp.py:87-110 (_silu_quant): gate = cols [0,K),
 * up = cols [K,2K); act = bf16(g / (1 + exp(-g))); v = bf16(act * up); rule
 * ceil_div448.  Rule 2 is the champion variant, mxfp8/swiglu_quant.py:54-66:
 * one bf16 rounding, v = bf16((g / (1 + exp(-g))) * up), then rp_ue8m0.
 * Outputs codes [rows, K] and logical scales [rows, K/32].                   */
void mxo_swiglu_mxfp8(const uint16_t* gate_up, int64_t rows, int64_t K, int rule,
                      uint8_t* codes, uint8_t* scales) {
  float v[32];
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t b = 0; b < K / 32; ++b) {
      for (int i = 0; i < 32; ++i) {
        float g = mxo_bf16_to_f32(gate_up[r * 2 * K + b * 32 + i]);
        float u = mxo_bf16_to_f32(gate_up[r * 2 * K + K + b * 32 + i]);
        if (rule == 2) {
          v[i] = bf16_round((g / (1.0f + mxo_exp(-g))) * u);
        } else {
          float act = bf16_round(g / (1.0f + mxo_exp(-g)));
          v[i] = bf16_round(act * u);
        }
      }
      quant_block32(v, rule, codes + r * K + b * 32, scales + r * (K / 32) + b);
    }
}

/* Scale swizzle used by the reference producers (mxfp8_mlp.py:107-110,122):
 * 128-row x 4-group tiles of 512 bytes.                                      */
int64_t mxo_swizzle_offset(int64_t r, int64_t g, int64_t K) {
  int64_t T = (K / 32 + 3) / 4;
  return (((r / 128 * T + g / 4) * 32 + r % 32) * 4 + (r % 128) / 32) * 4 + g % 4;
}

int64_t mxo_swizzle_size(int64_t rows, int64_t K) {
  return (rows + 127) / 128 * 128 * ((K / 32 + 3) / 4) * 4;
}

void mxo_swizzle_scales(const uint8_t* logical, int64_t rows, int64_t K, uint8_t* out) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t g = 0; g < K / 32; ++g) out[mxo_swizzle_offset(r, g, K)] = logical[r * (K / 32) + g];
}

/* -------------------------------------------- residual + RMSNorm producer */

/* Residual add + Gemma RMSNorm (+ MXFP8), mxfp6/mxfp8_norm_quant.py:15-39 and
 * mxfp6/gemma_norm.py:13-29.  Per row of N (N % 32 == 0):
 *   x      = f32(x) + f32(residual)        (no residual: x alone)
 *   summed = bf16(x)                        (the residual output)
 *   var    = (sum of x*x) / N               (sum order below)
 *   r      = 1 / sqrtf(var + eps)           (IEEE sqrt and divide; the reference's
 *                                            tl.rsqrt is an approximation that is not
 *                                            restated, so r is this build's definition)
 *   y      = bf16((x * r) * (f32(w) + 1))   (both products rounded, no FMA)
 * then either the bf16 y (gemma_norm) or the MXFP8 codes and E8M0 scales of y per
 * 32-block under `rule` (ceil_div448 in the reference, :27-33).
 * Sum order of the variance -- the order of the HIP kernel, which is what makes
 * the codes bit-exact: 256 workers; worker t owns the 8-element chunks
 * c = t, t + 256, ... and accumulates x*x over its chunks in chunk and element
 * order; the 64 workers of each group of 64 are combined as lane 0 of an xor
 * butterfly with distances 32, 16, 8, 4, 2, 1; the 4 group sums are added in
 * group order.                                                                  */
static float rms_sum_order(const float* x, int64_t N) {
  float part[256];
  for (int t = 0; t < 256; ++t) {
    float p = 0.0f;
    for (int64_t c = t; c < N / 8; c += 256)
      for (int k = 0; k < 8; ++k) p = p + x[c * 8 + k] * x[c * 8 + k];
    part[t] = p;
  }
  float total = 0.0f;
  for (int w = 0; w < 4; ++w) {
    float a[64], b[64];
    for (int l = 0; l < 64; ++l) a[l] = part[w * 64 + l];
    for (int off = 32; off >= 1; off >>= 1) {
      for (int l = 0; l < 64; ++l) b[l] = a[l] + a[l ^ off];
      memcpy(a, b, sizeof a);
    }
    total = w == 0 ? a[0] : total + a[0];
  }
  return total;
}

void mxo_rmsnorm_mx(const uint16_t* x, const uint16_t* residual, const uint16_t* weight, int64_t rows,
                    int64_t N, float eps, int rule, uint8_t* codes, uint8_t* scales, uint16_t* summed,
                    uint16_t* y_out) {
  float* v = (float*)malloc(sizeof(float) * (size_t)N);
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t i = 0; i < N; ++i) {
      float a = mxo_bf16_to_f32(x[r * N + i]);
      if (residual) a = a + mxo_bf16_to_f32(residual[r * N + i]);
      v[i] = a;
      if (summed) summed[r * N + i] = mxo_f32_to_bf16(a);
    }
    const float var = rms_sum_order(v, N) / (float)N;
    const float rs = 1.0f / sqrtf(var + eps);
    for (int64_t i = 0; i < N; ++i) v[i] = bf16_round((v[i] * rs) * (mxo_bf16_to_f32(weight[i]) + 1.0f));
    if (y_out) {
      for (int64_t i = 0; i < N; ++i) y_out[r * N + i] = mxo_f32_to_bf16(v[i]);
    } else {
      for (int64_t b = 0; b < N / 32; ++b) quant_block32(v + b * 32, rule, codes + r * N + b * 32, scales + r * (N / 32) + b);
    }
  }
  free(v);
}

/* ------------------------------------------------------------ block FP8 */

/* Per-token group-128 activation quantization, fp8/_quantize_kernel.py:8-18:
 * amax = max(max|x|, 1e-10); scale = amax / 448 (div_rn); q = clamp(x / scale,
 * +-448) -> E4M3; scales stored column-major S[g * M + m].                    */
void mxo_quant_block_fp8(const uint16_t* x, int64_t M, int64_t K, uint8_t* q, float* s_colmajor) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t g = 0; g < K / 128; ++g) {
      float amax = 0.0f;
      for (int i = 0; i < 128; ++i) { float a = fabsf(mxo_bf16_to_f32(x[m * K + g * 128 + i])); if (a > amax) amax = a; }
      if (!(amax >= 1e-10f)) amax = 1e-10f;
      float scale = amax / 448.0f;
      for (int i = 0; i < 128; ++i) {
        float y = mxo_bf16_to_f32(x[m * K + g * 128 + i]) / scale;
        y = fminf(fmaxf(y, -448.0f), 448.0f);
        q[m * K + g * 128 + i] = mxo_f32_to_e4m3(y);
      }
      s_colmajor[g * M + m] = scale;
    }
}

/* SiLU*up -> block-FP8, native/fp8_activation/activation.cu:33-59: fp32
 * sigmoid = 1/(1+exp(-g)), silu = g*sigmoid, v = silu*up (no bf16 rounding),
 * scale = max(amax/448, 1/(448*512)); q = clamp(v/scale, +-448) -> E4M3.
 * in [rows, 2H] -> q [rows, H], scales [rows, H/128] (or transposed).         */
void mxo_silu_mul_block_fp8(const uint16_t* in, int64_t rows, int64_t H, int transposed,
                            uint8_t* q, float* scales) {
  float v[128];
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t g = 0; g < H / 128; ++g) {
      float amax = 0.0f;
      for (int i = 0; i < 128; ++i) {
        float gt = mxo_bf16_to_f32(in[r * 2 * H + g * 128 + i]);
        float up = mxo_bf16_to_f32(in[r * 2 * H + H + g * 128 + i]);
        float sig = 1.0f / (1.0f + mxo_exp(-gt));
        v[i] = (gt * sig) * up;
        amax = fmaxf(amax, fabsf(v[i]));
      }
      float scale = fmaxf(amax / 448.0f, 1.0f / (448.0f * 512.0f));
      for (int i = 0; i < 128; ++i) {
        float y = fmaxf(-448.0f, fminf(v[i] / scale, 448.0f));
        q[r * H + g * 128 + i] = mxo_f32_to_e4m3(y);
      }
      scales[transposed ? g * rows + r : r * (H / 128) + g] = scale;
    }
}

/* Ordered block-FP8 reduction, fp8/ordered.py:137-149: given per-K128 raw
 * fp32 partial dots raw[g][m][n], total = fma(raw, sa[m,g]*sb[n/128,g], total)
 * in ascending g, then one bf16 rounding.  sa is column-major [K/128][M].      */
void mxo_block_fp8_ordered_reduce(const float* raw, const float* sa_colmajor, const float* sb,
                                  int64_t M, int64_t N, int64_t G, uint16_t* out) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      float total = 0.0f;
      for (int64_t g = 0; g < G; ++g) {
        float s = sa_colmajor[g * M + m] * sb[(n / 128) * G + g];
        total = fmaf(raw[(g * M + m) * N + n], s, total);
      }
      out[m * N + n] = mxo_f32_to_bf16(total);
    }
}

/* --------------------------------------------------------------- MXFP6 */

/* MXFP6 weight quantization per OCP MX v1.0 section 6.3 (the reference's
 * weights come from an external offline quantizer with no vectors in the
 * tree): shared exponent = floor(log2(amax)) - emax_elem (2 for E2M3, 4 for
 * E3M2), clamped to the E8M0 range; elements = saturating RNE(x / 2^exp);
 * an all-zero block gets code 0.  Outputs unpacked codes [rows, K].          */
void mxo_quant_mxfp6(const uint16_t* x, int64_t rows, int64_t K, int fmt,
                     uint8_t* codes, uint8_t* scales) {
  int emax = fmt == 2 ? 2 : 4;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t b = 0; b < K / 32; ++b) {
      float amax = 0.0f;
      for (int i = 0; i < 32; ++i) { float a = fabsf(mxo_bf16_to_f32(x[r * K + b * 32 + i])); if (a > amax) amax = a; }
      int e;
      if (amax == 0.0f) e = -127;
      else { int ex; frexpf(amax, &ex); e = (ex - 1) - emax; }
      if (e < -127) e = -127;
      if (e > 127) e = 127;
      float div = ldexpf(1.0f, e);
      for (int i = 0; i < 32; ++i) codes[r * K + b * 32 + i] = mxo_f32_to_fp6(mxo_bf16_to_f32(x[r * K + b * 32 + i]) / div, fmt);
      scales[r * (K / 32) + b] = (uint8_t)(e + 127);
    }
}

/* ----------------------------------------------------------- dequantize */

/* codes [rows, K] (fmt 0 = E4M3, 2 = E2M3, 3 = E3M2; FP6 unpacked) with
 * E8M0 scales [rows, K/32] -> fp32: value * 2^(s - 127)
 * (tests/native_mxfp6/test_mxfp8_sm120.py:55-56).                             */
void mxo_dequant_mx(const uint8_t* codes, const uint8_t* scales, int64_t rows, int64_t K, int fmt, float* out) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t k = 0; k < K; ++k) {
      uint8_t c = codes[r * K + k];
      float v = fmt == 0 ? mxo_e4m3_to_f32(c) : mxo_fp6_to_f32(c, fmt);
      out[r * K + k] = ldexpf(v, (int)scales[r * (K / 32) + k / 32] - 127);
    }
}

/* ------------------------------------------------------------------ MoE */

/* Token sort for routed experts (the contract of route_mxfp8_out,
 * mxfp6/moe_utils.py:205-255 and mxfp6/moe.py:651-669): routes r = t*topk+k
 * are grouped by expert id; within an expert they stay in ascending r.
 * expert_offsets[E+1] is the exclusive prefix of per-expert counts,
 * sorted_routes[pos] = r, inverse[r] = pos.  Ids outside [0, E) are dropped
 * (inverse = -1), which is how an expert_map marks non-local experts.        */
void mxo_moe_route(const int32_t* topk_ids, int64_t T, int64_t topk, int64_t E,
                   int32_t* sorted_routes, int64_t* expert_offsets, int32_t* inverse) {
  int64_t R = T * topk;
  memset(expert_offsets, 0, sizeof(int64_t) * (E + 1));
  for (int64_t r = 0; r < R; ++r) {
    int32_t e = topk_ids[r];
    if (e >= 0 && e < E) expert_offsets[e + 1]++;
  }
  for (int64_t e = 0; e < E; ++e) expert_offsets[e + 1] += expert_offsets[e];
  int64_t* fill = (int64_t*)malloc(sizeof(int64_t) * (E > 0 ? E : 1));
  for (int64_t e = 0; e < E; ++e) fill[e] = expert_offsets[e];
  for (int64_t r = 0; r < R; ++r) {
    int32_t e = topk_ids[r];
    if (e >= 0 && e < E) { int64_t p = fill[e]++; sorted_routes[p] = (int32_t)r; inverse[r] = (int32_t)p; }
    else inverse[r] = -1;
  }
  free(fill);
}

/* Weighted combine, mxfp6/moe.py:697-702 with the arithmetic of the reference's
 * check, tests/native_mxfp6/test_moe.py:243-247: each term y.float() * w is
 * rounded to binary32, terms are added in ascending k starting from zero, and
 * the sum is rounded once to bf16.  A dropped route contributes nothing.
 * y rows are bf16 in sorted order.                                           */
void mxo_moe_reduce(const uint16_t* y, const float* topk_weights, const int32_t* inverse,
                    int64_t T, int64_t topk, int64_t H, uint16_t* out) {
  for (int64_t t = 0; t < T; ++t)
    for (int64_t h = 0; h < H; ++h) {
      float acc = 0.0f;
      for (int64_t k = 0; k < topk; ++k) {
        int32_t p = inverse[t * topk + k];
        if (p < 0) continue;
        float term = mxo_bf16_to_f32(y[(int64_t)p * H + h]) * topk_weights[t * topk + k];
        acc = acc + term;
      }
      out[t * H + h] = mxo_f32_to_bf16(acc);
    }
}
