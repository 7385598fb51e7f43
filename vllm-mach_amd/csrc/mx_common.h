// Shared device helpers for the MI355X (gfx950) quantized-linear library.
//
// Every conversion here is a binary32 / integer operation sequence with
// round-to-nearest-even and no contraction (the library is compiled with
// -ffp-contract=off; fused steps call __builtin_fmaf explicitly), or a hardware
// conversion shown equal to such a sequence on every input, so codes and scales
// are bit-identical to a CPU evaluation of the same sequence.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "silu_math.h"
#include "silu_table.h"  // generated at build time (silu_table_gen.cpp)

namespace mxl {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// element formats understood by the scaled MFMA (cbsz / blgp operand)
enum Fmt : int { kE4M3 = 0, kE5M2 = 1, kE2M3 = 2, kE3M2 = 3 };

// E8M0 scale rules
enum Rule : int { kFloorCarry175 = 0, kCeilDiv448 = 1, kRpUe8m0 = 2 };

__device__ __forceinline__ uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

// Hardware pair conversions of gfx950.  Each was compared on the device with the
// integer sequence it replaces for all 2^32 binary32 inputs:
//  * v_cvt_pk_bf16_f32 (RNE) equals (u + 0x7FFF + bit16(u)) >> 16 on every non-NaN
//    input, overflow to infinity and subnormals included; a NaN keeps its sign and
//    the top of its payload.
//  * v_cvt_pk_fp8_f32 (OCP E4M3, RNE, no clamp) equals f32_to_e4m3 on every non-NaN
//    input (values from 464 up and infinities give sign | 0x7F); every NaN gives 0xFF.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// bf16 bits of (lo, hi) in the low / high half; NaN payloads pass through
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

// round-to-nearest-even binary32 -> bf16, NaN -> 0x7FC0
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return f != f ? (uint16_t)0x7FC0 : (uint16_t)cvt_pk_bf16(f, 0.0f);
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// bf16_round of a pair in one conversion, without NaN canonicalization: a NaN stays
// a NaN of unspecified sign and payload (for values whose NaNs are all coded alike)
__device__ __forceinline__ void bf16_round2_nan_any(float& lo, float& hi) {
  const uint32_t w = cvt_pk_bf16(lo, hi);
  lo = u2f(w << 16);
  hi = u2f(w & 0xFFFF0000u);
}

// Four binary32 values -> four E4M3 codes (byte i = value i), equal to f32_to_e4m3 on
// every input: a positive NaN, which the instruction would code 0xFF, is first replaced
// by +inf (code 0x7F, as 480 and above): as signed integers positive NaNs are exactly
// the values above +inf's bits, so one integer min does it.
__device__ __forceinline__ float e4m3_pos_nan_to_inf(float y) {
  const int32_t b = (int32_t)f2u(y);
  return u2f((uint32_t)(b < (int32_t)0x7F800000 ? b : (int32_t)0x7F800000));
}
// (exact unless an input is a positive NaN)
__device__ __forceinline__ uint32_t e4m3x4_raw(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  return e4m3x4_raw(e4m3_pos_nan_to_inf(a), e4m3_pos_nan_to_inf(b), e4m3_pos_nan_to_inf(c),
                    e4m3_pos_nan_to_inf(d));
}

// binary32 -> E4M3 ("fn") with torch's cast semantics: RNE onto the E4M3
// grid; magnitudes that round past 448, or are >= 480, give the NaN code.
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
  uint32_t u = f2u(f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  if (a >= 0x43F00000u) return sign | 0x7Fu;
  if (a < 0x3C800000u) return sign | (uint32_t)__builtin_rintf(u2f(a) * 512.0f);
  uint32_t odd = (a >> 20) & 1u;
  return sign | ((a - (120u << 23) + 0x7FFFFu + odd) >> 20);
}

// E4M3 ("fn") code -> binary32 (exact; 0x7F / 0xFF decode as NaN).
__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
  const uint32_t e = (c >> 3) & 0xFu, m = c & 7u;
  const float sgn = (c & 0x80u) ? -1.0f : 1.0f;
  if (e == 0xFu && m == 7u) return __builtin_nanf("");
  if (e == 0u) return sgn * __builtin_ldexpf((float)m, -9);
  return sgn * __builtin_ldexpf((float)(8u + m), (int)e - 10);
}

// binary32 -> FP6 code (fmt 2 = E2M3, 3 = E3M2; bit 5 = sign), OCP MX v1.0:
// round-to-nearest-even, saturating to the largest normal; FP6 has no NaN, and a
// NaN gives the signed zero code.
template <int FMT>
__device__ __forceinline__ uint32_t f32_to_fp6(float f) {
  constexpr int MB = FMT == kE2M3 ? 3 : 2, BIAS = FMT == kE2M3 ? 1 : 3;
  const uint32_t u = f2u(f);
  const uint32_t sign = (u >> 26) & 0x20u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign;
  uint32_t code;
  if (a < ((uint32_t)(128 - BIAS) << 23)) {
    code = (uint32_t)__builtin_rintf(__builtin_ldexpf(u2f(a), BIAS - 1 + MB));  // subnormal grid
  } else {
    constexpr int SH = 23 - MB;
    const uint32_t odd = (a >> SH) & 1u;
    code = (a - ((uint32_t)(127 - BIAS) << 23) + ((1u << (SH - 1)) - 1u) + odd) >> SH;
  }
  return sign | (code > 31u ? 31u : code);
}

// E8M0 code of the floor_carry175 rule from the bf16 bits of the block amax
__device__ __forceinline__ uint32_t scale_floor_carry175(uint32_t amax_bf16) {
  uint32_t e = (((amax_bf16 + 32u) & 0xFF80u) >> 7) & 0xFFu;
  return e == 0 ? 0u : (uint32_t)((int)e - 8) & 0xFFu;
}

// power-of-two bits (exponent field only) of the ceil_div448 rule
__device__ __forceinline__ uint32_t pow2_ceil_div448(float amax) {
  float raw = amax / 448.0f;
  if (!(raw >= 1.0e-30f)) raw = 1.0e-30f;
  return (f2u(raw) + 0x007FFFFFu) & 0x7F800000u;
}

// rp_ue8m0 (FlashInfer's mxfp8_quantize convention, mxfp8/swiglu_quant.py:58-66):
// E8M0 code of raw = amax * (1/448) rounded toward +inf, saturating at 254 (raw is
// never negative or NaN: the amax skips NaNs); 2^-127 is the subnormal 0x00400000.
__device__ __forceinline__ uint32_t e8m0_rp(float amax) {
  const uint32_t u = f2u(amax * (1.0f / 448.0f));
  const uint32_t e = u >> 23, up = e + ((u & 0x7FFFFFu) != 0u);
  const uint32_t sub = u <= 0x00400000u ? 0u : 1u;
  const uint32_t s = e == 0u ? sub : (up > 254u ? 254u : up);
  return u >= 0x7F800000u ? 254u : s;
}
// its element multiplier: 2^(127 - s); 0 for s = 0 and for s = 254 (2^-127 is subnormal,
// flushed by the reference's reciprocal)
__device__ __forceinline__ float e8m0_rp_inverse(uint32_t s) {
  return (s == 0u || s == 254u) ? 0.0f : u2f((254u - s) << 23);
}

// SwiGLU of eight (gate, up) pairs: act = bf16(g / (1 + exp(-g))) and v = bf16(act * u)
// (mxfp8_mlp.py:96-97), or for the rp_ue8m0 rule v = bf16((g / (1 + exp(-g))) * u)
// (swiglu_quant.py:56-57).  A NaN act makes a NaN v, and quant8x4<RULE, true> codes every
// NaN v as the canonical one, so the pair roundings leave NaN sign and payload as they come.
template <int RULE, int N = 8>
__device__ __forceinline__ void swiglu8(const float* g, const float* u, float* v) {
#pragma unroll
  for (int i = 0; i < N; i += 2) {
    float a0 = mx_silu(g[i]), a1 = mx_silu(g[i + 1]);
    if (RULE != kRpUe8m0) bf16_round2_nan_any(a0, a1);
    v[i] = a0 * u[i];
    v[i + 1] = a1 * u[i + 1];
    bf16_round2_nan_any(v[i], v[i + 1]);
  }
}

// The E8M0 code of a block from its amax (every lane of the block passes the same
// amax) and the lane's N codes (N % 4 == 0) packed into N / 4 dwords: quant8x4's
// arithmetic (below) for any number of the block's values per lane.  NAN_ANY as there.
template <int RULE, bool NAN_ANY, int N>
__device__ __forceinline__ uint32_t quant_block_codes(const float* v, float amax, uint32_t* packed) {
  static_assert(N % 4 == 0, "whole code dwords");
  uint32_t s;
  float y[N];
  if (RULE == kRpUe8m0) {
    // min(max(v * inverse, -448), 448): no NaN is left for the conversion
    s = e8m0_rp(amax);
    const float inv = e8m0_rp_inverse(s);
#pragma unroll
    for (int i = 0; i < N; ++i) y[i] = __builtin_fminf(__builtin_fmaxf(v[i] * inv, -448.0f), 448.0f);
#pragma unroll
    for (int i = 0; i < N / 4; ++i) packed[i] = e4m3x4_raw(y[4 * i], y[4 * i + 1], y[4 * i + 2], y[4 * i + 3]);
    return s;
  }
  if (RULE == kFloorCarry175) {
    s = scale_floor_carry175(f2u(amax) >> 16);
    const int e2 = 127 - (int)s;
#pragma unroll
    for (int i = 0; i < N; ++i) y[i] = __builtin_ldexpf(v[i], e2);
  } else {
    const uint32_t bits = pow2_ceil_div448(amax);
    s = bits >> 23;
    const float mul = 1.0f / u2f(bits);
    if (NAN_ANY && bits == 0x7F800000u) {
      // an infinite amax: mul = 0 and inf * 0 makes a NaN of the multiply's own sign,
      // coded by f32_to_e4m3 from the product of the canonical values
#pragma unroll
      for (int i = 0; i < N; ++i) y[i] = (v[i] != v[i] ? u2f(0x7FC00000u) : v[i]) * mul;
#pragma unroll
      for (int i = 0; i < N / 4; ++i)
        packed[i] = f32_to_e4m3(y[4 * i]) | f32_to_e4m3(y[4 * i + 1]) << 8 | f32_to_e4m3(y[4 * i + 2]) << 16 |
                    f32_to_e4m3(y[4 * i + 3]) << 24;
      return s;
    }
#pragma unroll
    for (int i = 0; i < N; ++i) y[i] = v[i] * mul;
  }
  if (NAN_ANY) {
    // every NaN (and every value from 480 up) -> 480 -> 0x7F
#pragma unroll
    for (int i = 0; i < N; ++i) y[i] = __builtin_fminf(y[i], 480.0f);
#pragma unroll
    for (int i = 0; i < N / 4; ++i) packed[i] = e4m3x4_raw(y[4 * i], y[4 * i + 1], y[4 * i + 2], y[4 * i + 3]);
  } else {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) packed[i] = e4m3x4(y[4 * i], y[4 * i + 1], y[4 * i + 2], y[4 * i + 3]);
  }
  return s;
}

// The bf16 magnitude bits of the largest |x| over N raw bf16 pairs.  SKIP_NAN: of the
// largest non-NaN |x| (0 when all are NaN), equal to the bf16 bits of the quieted-float
// amax -- per 16-bit half, |x| + 0x7F keeps every non-NaN magnitude (at most +inf's
// 0x7F80) below 0x8000 and moves every NaN magnitude (0x7F81 .. 0x7FFF) to 0x8000 and
// above, negative as a signed half, so a signed packed max skips the NaNs (the halves
// never carry into each other).  Otherwise NaNs count, so a result above 0x7F80 says
// that a NaN is present.
typedef short i16x2_t __attribute__((ext_vector_type(2)));
template <int N, bool SKIP_NAN>
__device__ __forceinline__ uint32_t amax_bf16_bits(const uint32_t* d) {
  const uint32_t bias = SKIP_NAN ? 0x007F007Fu : 0u;
  i16x2_t m = __builtin_bit_cast(i16x2_t, bias);
#pragma unroll
  for (int i = 0; i < N; ++i)
    m = __builtin_elementwise_max(m, __builtin_bit_cast(i16x2_t, (d[i] & 0x7FFF7FFFu) + bias));
  return (uint32_t)((m[0] > m[1] ? m[0] : m[1]) - (int)(bias & 0xFFu));
}

// 4 N raw bf16 values (2 N pairs) -> N dwords of E4M3 codes divided by 2^(s - 127),
// s < 255: v_cvt_scalef32_pk_fp8_bf16 divides by the power of two its scale operand's
// exponent field names and rounds once, which equals f32_to_e4m3(ldexpf(x, 127 - s)) for
// every bf16 x and s < 255 (checked on the device for all 65536 x 255 pairs) except
// positive NaNs, which it codes 0xFF.  NAN_FIX turns those into +inf first (code 0x7F),
// the signed packed min with +inf's bits doing for both halves what e4m3_pos_nan_to_inf
// does; without it the caller guarantees that no input is a NaN.
template <int N, bool NAN_FIX>
__device__ __forceinline__ void codes_bf16_scaled(const uint32_t* d, uint32_t s, uint32_t* packed) {
  const float scale = u2f(s << 23);
  const i16x2_t inf2 = __builtin_bit_cast(i16x2_t, 0x7F807F80u);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    i16x2_t lo = __builtin_bit_cast(i16x2_t, d[2 * i]), hi = __builtin_bit_cast(i16x2_t, d[2 * i + 1]);
    if (NAN_FIX) {
      lo = __builtin_elementwise_min(lo, inf2);
      hi = __builtin_elementwise_min(hi, inf2);
    }
    // both 16-bit halves of the result are written, so the first conversion's "old"
    // operand is any register: its own source
    i16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(lo, __builtin_bit_cast(bf16x2_t, lo), scale, false);
    c = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(c, __builtin_bit_cast(bf16x2_t, hi), scale, true);
    packed[i] = __builtin_bit_cast(uint32_t, c);
  }
}

// Quantize one 32-element block held by 4 consecutive lanes (8 values each,
// lane (tid & 3) owns elements [8 (tid & 3), +8)).  The block amax is an
// xor-shuffle max over the 4 lanes (order-free, so identical to a serial max).
// Returns the E8M0 code (valid in every lane) and the lane's 8 codes packed
// into two dwords.  The codes equal f32_to_e4m3 of the scaled values.
// NAN_ANY: the caller's NaNs stand for the canonical positive NaN whatever their
// sign and payload (values that bf16_round2_nan_any produced), so every NaN is
// coded 0x7F, as f32_to_e4m3 codes the canonical one.
template <int RULE, bool NAN_ANY = false>
__device__ __forceinline__ uint32_t quant8x4(const float* v, uint32_t* packed) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
  amax = __builtin_fmaxf(amax, __shfl_xor(amax, 1, 4));
  amax = __builtin_fmaxf(amax, __shfl_xor(amax, 2, 4));
  return quant_block_codes<RULE, NAN_ANY, 8>(v, amax, packed);
}

// Unpack 8 bf16 from a 16-byte vector into floats
__device__ __forceinline__ void bf16x8_to_f32(uint4 q, float* f) {
  uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = u2f(w[i] << 16);
    f[2 * i + 1] = u2f(w[i] & 0xFFFF0000u);
  }
}

// Quiet signaling NaNs (sign, payload top bits and subnormals are kept).  An amax
// over raw inputs needs it: in IEEE mode v_max_f32 / v_max3_f32 return a NaN when an
// operand is a signaling NaN, where the block amax skips every NaN.
__device__ __forceinline__ void quiet8(float* f) {
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = __builtin_canonicalizef(f[i]);
}

// quant8x4 of 8 raw bf16 values (one 16-byte load; four lanes per block, lane (tid & 3)
// owning elements [8 (tid & 3), +8)), equal to bf16x8_to_f32 + quiet8 + quant8x4<RULE>:
// where the block's scale is a power of two (rules 0 and 1) below E8M0 code 255 and no
// value of the block is a NaN, the codes come straight from the bf16 pairs
// (amax_bf16_bits, codes_bf16_scaled); other blocks take the binary32 arithmetic.  The
// condition is the block's, so the four lanes of a block take the same path.
template <int RULE>
__device__ __forceinline__ uint32_t quant8x4_bf16(uint4 raw, uint32_t* packed) {
  if constexpr (RULE != kRpUe8m0) {
    const uint32_t d[4] = {raw.x, raw.y, raw.z, raw.w};
    uint32_t mb = amax_bf16_bits<4, false>(d);
    mb = __builtin_elementwise_max(mb, (uint32_t)__shfl_xor((int)mb, 1, 4));
    mb = __builtin_elementwise_max(mb, (uint32_t)__shfl_xor((int)mb, 2, 4));
    const uint32_t sf = RULE == kFloorCarry175 ? scale_floor_carry175(mb) : pow2_ceil_div448(u2f(mb << 16)) >> 23;
    if (mb <= 0x7F80u && sf < 255u) {
      codes_bf16_scaled<2, false>(d, sf, packed);
      return sf;
    }
  }
  float v[8];
  bf16x8_to_f32(raw, v);
  quiet8(v);
  return quant8x4<RULE>(v, packed);
}

// SwiGLU activations from the table: per 16-bit half of a gate dword, (g & 0x7FFF) -
// (kSiluELo << 7) is the table offset when below kSiluSpan (gates under the range wrap
// around to large offsets), and bit 15 moved to bit 12 adds kSiluSpan (4096) for a
// negative gate.  silu_offsets returns the pair of offsets; the lane's gates all lie in
// the table when the largest offset of its dwords is below kSiluSpan.
static_assert(kSiluSpan == 4096, "the sign bit selects the negative half by one shift");
__device__ __forceinline__ uint32_t silu_offsets(uint32_t d) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  const u16x2 lo = __builtin_bit_cast(u16x2, (kSiluELo << 7) | (kSiluELo << 23));
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, d & 0x7FFF7FFFu) - lo);
}
__device__ __forceinline__ bool silu_in_table(uint4 graw) {
  const uint32_t o[4] = {silu_offsets(graw.x), silu_offsets(graw.y), silu_offsets(graw.z), silu_offsets(graw.w)};
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) m = __builtin_elementwise_max(m, (o[i] & 0xFFFFu)), m = __builtin_elementwise_max(m, o[i] >> 16);
  return m < kSiluSpan;
}

// bf16x8_to_f32 + swiglu8<RULE> + quant8x4<RULE, true> of a lane's 8 (gate, up) pairs for
// rules 0 and 1, with each activation bf16(mx_silu(g)) read from the table staged in LDS
// (tab) -- the caller has checked silu_in_table for the four lanes of the block -- and
// the codes of power-of-two-scaled NaN-free blocks straight from the bf16 products
// (amax_bf16_bits, codes_bf16_scaled); other blocks take the binary32 arithmetic.
template <int RULE>
__device__ __forceinline__ uint32_t swiglu_quant8_table(uint4 graw, uint4 uraw, const uint16_t* tab, uint32_t* packed) {
  static_assert(RULE == kFloorCarry175 || RULE == kCeilDiv448, "the table holds the bf16-rounded activation");
  const uint32_t gd[4] = {graw.x, graw.y, graw.z, graw.w}, ud[4] = {uraw.x, uraw.y, uraw.z, uraw.w};
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t o = silu_offsets(gd[i]) + ((gd[i] >> 3) & 0x10001000u);
    const float a0 = u2f((uint32_t)tab[o & 0xFFFFu] << 16), a1 = u2f((uint32_t)tab[o >> 16] << 16);
    w[i] = cvt_pk_bf16(a0 * u2f(ud[i] << 16), a1 * u2f(ud[i] & 0xFFFF0000u));
  }
  uint32_t mb = amax_bf16_bits<4, false>(w);
  mb = __builtin_elementwise_max(mb, (uint32_t)__shfl_xor((int)mb, 1, 4));
  mb = __builtin_elementwise_max(mb, (uint32_t)__shfl_xor((int)mb, 2, 4));
  const uint32_t sf = RULE == kFloorCarry175 ? scale_floor_carry175(mb) : pow2_ceil_div448(u2f(mb << 16)) >> 23;
  if (mb <= 0x7F80u && sf < 255u) {
    codes_bf16_scaled<2, false>(w, sf, packed);
    return sf;
  }
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = u2f(w[i] << 16);
    v[2 * i + 1] = u2f(w[i] & 0xFFFF0000u);
  }
  return quant8x4<RULE, true>(v, packed);
}

// Block-FP8 activation quantization of one 128-element group held by 16 consecutive
// lanes (8 quieted values each; fp8/_quantize_kernel.py:7-18): the group amax by an
// xor-shuffle max (order-free), floored at 1e-10, scale = amax / 448, codes =
// E4M3(clamp(v / scale, +-448)).  Returns the scale; the lane's codes in w[0], w[1].
__device__ __forceinline__ float block_fp8_quant8(const float* v, uint32_t* w) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = __builtin_fmaxf(m, __builtin_fabsf(v[i]));
#pragma unroll
  for (int d = 8; d >= 1; d >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, d, 16));
  m = __builtin_fmaxf(m, 1e-10f);
  const float scale = m / 448.0f;
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = __builtin_fminf(__builtin_fmaxf(v[i] / scale, -448.0f), 448.0f);
  // the clamp leaves no NaN: the hardware conversion equals f32_to_e4m3 here
  w[0] = e4m3x4_raw(y[0], y[1], y[2], y[3]);
  w[1] = e4m3x4_raw(y[4], y[5], y[6], y[7]);
  return scale;
}

}  // namespace mxl

// ---------------------------------------------------------------- host side

#define MXL_OK 0
#define MXL_EINVAL -1
#define MXL_EHIP -2
#define MXL_EUNSUPPORTED -3

namespace mxl {
void set_error(const char* fmt, ...);
}

#define MXL_CHECK_ARG(cond, ...)           \
  do {                                     \
    if (!(cond)) {                         \
      ::mxl::set_error(__VA_ARGS__);       \
      return MXL_EINVAL;                   \
    }                                      \
  } while (0)

#define MXL_CHECK_LAUNCH(what)                                                       \
  do {                                                                               \
    hipError_t e_ = hipGetLastError();                                               \
    if (e_ != hipSuccess) {                                                          \
      ::mxl::set_error("%s: launch failed: %s", what, hipGetErrorString(e_));       \
      return MXL_EHIP;                                                               \
    }                                                                                \
  } while (0)
