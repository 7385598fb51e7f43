// Activation quantizers and fused producers for gfx950.
//
//  * MXFP8 dynamic quantization (E4M3 codes, E8M0 scale per 32 along K)
//  * SwiGLU -> MXFP8 producer (bf16 SiLU, bf16 product, ceil_div448 scales)
//  * block-FP8 per-token group-128 quantization (fp32 scales, column-major)
//  * SiLU*up -> block-FP8 producer
//
// All four are HBM-bound elementwise passes: four lanes own one 32-element MX
// block and 16 lanes own one 128-element group, each lane holding 8 values
// from one 16-byte load; the amax is an xor-shuffle max inside the group.  Loads and
// stores are 16-byte vectors; consecutive threads walk consecutive blocks of
// a row so every wavefront access is one contiguous span.
#include <algorithm>

#include "mx_common.h"

namespace mxl {

// Lane -> (row, block) of a G-lanes-per-block mapping (G = 4 for 32-element MX
// blocks, 16 for 128-element groups) in 32-bit arithmetic: the host keeps the lane
// count below 2^31 (lanes_fit).  Lanes past the end shadow the last block with
// live = false, so every lane takes part in the block's shuffles.
template <int G>
struct BlockLane {
  uint32_t row, blk;
  int sub;
  bool live;
  __device__ __forceinline__ BlockLane(uint32_t blocks_per_row, uint32_t blocks) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    sub = (int)(t % G);
    live = t / G < blocks;
    const uint32_t id = live ? t / G : blocks - 1;
    row = id / blocks_per_row;
    blk = id - row * blocks_per_row;
  }
};

// --------------------------------------------------------------- MXFP8 quant

// Four lanes own one 32-element block (8 values, one 16-byte load each), so a
// decode-sized launch still spreads over enough lanes to hide latency.
__device__ __forceinline__ int64_t swizzle_offset(int64_t r, int64_t g, int64_t K);

template <int RULE, bool SWIZZLED = false>
__global__ __launch_bounds__(256) void quant_mxfp8_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                          uint8_t* __restrict__ codes,
                                                          uint8_t* __restrict__ scales, int64_t M,
                                                          int64_t K) {
  const int64_t blocks_per_row = K / 32;
  const BlockLane<4> bl((uint32_t)blocks_per_row, (uint32_t)(M * blocks_per_row));
  const int sub = bl.sub;
  const bool live = bl.live;
  const int64_t row = bl.row, blk = bl.blk;
  uint32_t packed[2];
  const uint32_t s = quant8x4_bf16<RULE>(*reinterpret_cast<const uint4*>(x + row * ldx + blk * 32 + sub * 8), packed);
  if (!live) return;
  *reinterpret_cast<uint2*>(codes + row * K + blk * 32 + sub * 8) = make_uint2(packed[0], packed[1]);
  if (sub == 0) scales[SWIZZLED ? swizzle_offset(row, blk, K) : row * blocks_per_row + blk] = (uint8_t)s;
}

// ------------------------------------------------------------ MXFP6 weights

// OCP MX v1.0 section 6.3 quantization of bf16 weights to MXFP6: shared exponent
// e = floor(log2(amax)) - emax (2 for E2M3, 4 for E3M2), clamped to the E8M0
// range (an all-zero block gets code 0), elements = saturating RNE(x / 2^e),
// packed four 6-bit codes per three bytes (little-endian bit stream).  Four
// lanes own a 32-element block; each writes its 8 codes as 6 bytes.
template <int FMT>
__global__ __launch_bounds__(256) void quant_mxfp6_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                          uint8_t* __restrict__ packed,
                                                          uint8_t* __restrict__ scales, int64_t M, int64_t K) {
  const int64_t blocks_per_row = K / 32;
  const BlockLane<4> bl((uint32_t)blocks_per_row, (uint32_t)(M * blocks_per_row));
  const int sub = bl.sub;
  const bool live = bl.live;
  const int64_t row = bl.row, blk = bl.blk;
  float v[8];
  bf16x8_to_f32(*reinterpret_cast<const uint4*>(x + row * ldx + blk * 32 + sub * 8), v);
  quiet8(v);
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
  amax = __builtin_fmaxf(amax, __shfl_xor(amax, 1, 4));
  amax = __builtin_fmaxf(amax, __shfl_xor(amax, 2, 4));
  constexpr int EMAX = FMT == kE2M3 ? 2 : 4;
  // floor(log2(amax)) from the exponent field; zero and subnormal amax (floor(log2) <= -127) clamp to -127
  const int ef = (int)((f2u(amax) >> 23) & 0xFFu);
  int e = ef == 0 ? -127 : ef - 127 - EMAX;
  e = e < -127 ? -127 : (e > 127 ? 127 : e);
  uint32_t c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = f32_to_fp6<FMT>(__builtin_ldexpf(v[i], -e));
  const uint32_t w0 = c[0] | (c[1] << 6) | (c[2] << 12) | (c[3] << 18);
  const uint32_t w1 = c[4] | (c[5] << 6) | (c[6] << 12) | (c[7] << 18);
  if (!live) return;
  uint16_t* dst = reinterpret_cast<uint16_t*>(packed + row * (K * 3 / 4) + blk * 24 + sub * 6);
  dst[0] = (uint16_t)w0;
  dst[1] = (uint16_t)((w0 >> 16) | ((w1 & 0xFFu) << 8));
  dst[2] = (uint16_t)(w1 >> 8);
  if (sub == 0) scales[row * blocks_per_row + blk] = (uint8_t)(e + 127);
}

// Two-limb MXFP8: hi = MXFP8(x), residual = bf16(x - deq(hi)), res = MXFP8(residual),
// both under RULE (the contract of mxfp8/dual.py:45-50; the quantizer itself is
// this build's definition).  Same lane mapping as quant_mxfp8_kernel.
template <int RULE>
__global__ __launch_bounds__(256) void quant_mxfp8_dual_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                               uint8_t* __restrict__ hi, uint8_t* __restrict__ s_hi,
                                                               uint8_t* __restrict__ res,
                                                               uint8_t* __restrict__ s_res, int64_t M, int64_t K) {
  const int64_t blocks_per_row = K / 32;
  const BlockLane<4> bl((uint32_t)blocks_per_row, (uint32_t)(M * blocks_per_row));
  const int sub = bl.sub;
  const bool live = bl.live;
  const int64_t row = bl.row, blk = bl.blk;
  float v[8], rv[8];
  bf16x8_to_f32(*reinterpret_cast<const uint4*>(x + row * ldx + blk * 32 + sub * 8), v);
  quiet8(v);
  uint32_t ph[2], pr[2];
  const uint32_t sh = quant8x4<RULE>(v, ph);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float deq = __builtin_ldexpf(e4m3_to_f32((ph[i >> 2] >> (8 * (i & 3))) & 0xFFu), (int)sh - 127);
    rv[i] = bf16_round(v[i] - deq);
  }
  const uint32_t sr = quant8x4<RULE>(rv, pr);
  if (!live) return;
  const int64_t off = row * K + blk * 32 + sub * 8;
  *reinterpret_cast<uint2*>(hi + off) = make_uint2(ph[0], ph[1]);
  *reinterpret_cast<uint2*>(res + off) = make_uint2(pr[0], pr[1]);
  if (sub == 0) {
    s_hi[row * blocks_per_row + blk] = (uint8_t)sh;
    s_res[row * blocks_per_row + blk] = (uint8_t)sr;
  }
}

// ------------------------------------------------------------ SwiGLU -> MXFP8

__device__ __forceinline__ int64_t swizzle_offset(int64_t r, int64_t g, int64_t K) {
  const int64_t T = (K / 32 + 3) / 4;
  return (((r / 128 * T + g / 4) * 32 + r % 32) * 4 + (r % 128) / 32) * 4 + g % 4;
}

// The workgroup's threads stride over the items (four lanes per 32-block, 8 values
// each).  TABLE (rules 0 and 1, 1024 threads): the workgroup first stages the SiLU table
// (16 KiB) in LDS, and a wave whose gates all lie in it reads the activations from it
// instead of evaluating exp and the division.  Without it (small launches, where the
// staging costs more than it saves, and rule 2) 256 threads, one item each.
constexpr int kSwigluThreads = 1024;
// the table pays from about half a 1024-thread workgroup's items per CU
constexpr int64_t kSwigluTableItemsPerCu = 512;
int cu_count();  // compute units of the current device (gemm_stream.hip)
template <int RULE, bool SWIZZLED, bool TABLE>
__global__ __launch_bounds__(TABLE ? kSwigluThreads : 256) void swiglu_mxfp8_kernel(const uint16_t* __restrict__ gate_up,
                                                                                    uint8_t* __restrict__ codes,
                                                                                    uint8_t* __restrict__ scales,
                                                                                    int64_t M, int64_t K) {
  static_assert(!TABLE || RULE != kRpUe8m0, "the table holds the bf16-rounded activation of rules 0 and 1");
  constexpr bool TAB = TABLE;
  __shared__ __attribute__((aligned(16))) uint16_t tab[TAB ? kSiluEntries : 8];
  if constexpr (TAB) {
    for (uint32_t i = threadIdx.x; i < kSiluEntries / 8; i += blockDim.x)
      reinterpret_cast<uint4*>(tab)[i] = reinterpret_cast<const uint4*>(kSiluAct)[i];
    __syncthreads();
  }
  // lanes are indexed in 32 bits (the host bounds the item count)
  const uint32_t blocks_per_row = (uint32_t)(K / 32), items = (uint32_t)M * blocks_per_row * 4;
  // the same trip count for every thread of the workgroup; items past the end redo the
  // last block without storing, so the four lanes of a block stay together
  for (uint32_t base = blockIdx.x * blockDim.x; base < items; base += gridDim.x * blockDim.x) {
    const uint32_t t = base + threadIdx.x;
    const bool live = t < items;
    const uint32_t it = live ? t : items - 4 + (t & 3);
    const int sub = (int)(it & 3);
    const uint32_t id = it >> 2;
    const int64_t row = id / blocks_per_row, blk = id - (uint32_t)row * blocks_per_row;
    const int64_t off = row * 2 * K + blk * 32 + sub * 8;
    const uint4 graw = *reinterpret_cast<const uint4*>(gate_up + off);
    const uint4 uraw = *reinterpret_cast<const uint4*>(gate_up + off + K);
    uint32_t packed[2], s = 0;
    bool done = false;
    if constexpr (TAB) {
      if (__builtin_amdgcn_ballot_w64(!silu_in_table(graw)) == 0) {
        s = swiglu_quant8_table<RULE>(graw, uraw, tab, packed);
        done = true;
      }
    }
    if (!done) {
      float g[8], u[8], v[8];
      bf16x8_to_f32(graw, g);
      bf16x8_to_f32(uraw, u);
      swiglu8<RULE>(g, u, v);
      s = quant8x4<RULE, true>(v, packed);
    }
    if (live) {
      *reinterpret_cast<uint2*>(codes + row * K + blk * 32 + sub * 8) = make_uint2(packed[0], packed[1]);
      if (sub == 0) {
        if (SWIZZLED)
          scales[swizzle_offset(row, blk, K)] = (uint8_t)s;
        else
          scales[row * blocks_per_row + blk] = (uint8_t)s;
      }
    }
  }
}

// Zero the padding bytes of a swizzled scale buffer (rows beyond M inside the
// last 128-row tile and groups beyond K/32 inside the last 4-group tile), so
// the buffer content is a pure function of the input.
__global__ void swizzle_pad_kernel(uint8_t* __restrict__ scales, int64_t M, int64_t K, int64_t total) {
  const int64_t off = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (off >= total) return;
  // invert the map: off = (((rt*T + gt)*32 + r32)*4 + r4)*4 + g4
  const int64_t T = (K / 32 + 3) / 4;
  int64_t t = off;
  const int64_t g4 = t % 4; t /= 4;
  const int64_t r4 = t % 4; t /= 4;
  const int64_t r32 = t % 32; t /= 32;
  const int64_t gt = t % T, rt = t / T;
  const int64_t r = rt * 128 + r4 * 32 + r32, g = gt * 4 + g4;
  if (r >= M || g >= K / 32) scales[off] = 0;
}

// Logical [R, K/32] E8M0 -> the swizzled layout, padding zeroed: one thread per
// byte of the swizzled buffer (the inverse map of swizzle_offset).
__global__ void swizzle_scales_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t R,
                                      int64_t K, int64_t total) {
  const int64_t off = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (off >= total) return;
  const int64_t T = (K / 32 + 3) / 4;
  int64_t t = off;
  const int64_t g4 = t % 4; t /= 4;
  const int64_t r4 = t % 4; t /= 4;
  const int64_t r32 = t % 32; t /= 32;
  const int64_t gt = t % T, rt = t / T;
  const int64_t r = rt * 128 + r4 * 32 + r32, g = gt * 4 + g4;
  dst[off] = (r < R && g < K / 32) ? src[r * (K / 32) + g] : (uint8_t)0;
}

// ------------------------------------------------------- block-FP8 quantizer

// 16 lanes own one 128-element group; each lane holds 8 consecutive values.
__device__ __forceinline__ float group16_amax(float m) {
#pragma unroll
  for (int d = 8; d >= 1; d >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, d, 16));
  return m;
}

__global__ __launch_bounds__(256) void quant_block_fp8_kernel(const uint16_t* __restrict__ x,
                                                              uint8_t* __restrict__ q,
                                                              float* __restrict__ s_colmajor,
                                                              int64_t M, int64_t K) {
  const BlockLane<16> bl((uint32_t)(K / 128), (uint32_t)(M * (K / 128)));
  const int sub = bl.sub;
  const bool live = bl.live;
  const int64_t row = bl.row, col = bl.blk;
  float v[8];
  bf16x8_to_f32(*reinterpret_cast<const uint4*>(x + row * K + col * 128 + sub * 8), v);
  quiet8(v);
  uint32_t w[2];
  const float scale = block_fp8_quant8(v, w);
  if (!live) return;
  *reinterpret_cast<uint2*>(q + row * K + col * 128 + sub * 8) = make_uint2(w[0], w[1]);
  if (sub == 0) s_colmajor[col * M + row] = scale;
}

template <bool TRANSPOSED>
__global__ __launch_bounds__(256) void silu_mul_block_fp8_kernel(const uint16_t* __restrict__ in,
                                                                 uint8_t* __restrict__ q,
                                                                 float* __restrict__ scales,
                                                                 int64_t rows, int64_t H) {
  const BlockLane<16> bl((uint32_t)(H / 128), (uint32_t)(rows * (H / 128)));
  const int sub = bl.sub;
  const bool live = bl.live;
  const int64_t row = bl.row, col = bl.blk;
  float gt[8], up[8], v[8];
  bf16x8_to_f32(*reinterpret_cast<const uint4*>(in + row * 2 * H + col * 128 + sub * 8), gt);
  bf16x8_to_f32(*reinterpret_cast<const uint4*>(in + row * 2 * H + H + col * 128 + sub * 8), up);
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float sig = 1.0f / (1.0f + mx_exp(-gt[i]));
    v[i] = (gt[i] * sig) * up[i];
    m = __builtin_fmaxf(m, __builtin_fabsf(v[i]));
  }
  m = group16_amax(m);
  const float scale = __builtin_fmaxf(m / 448.0f, 1.0f / (448.0f * 512.0f));
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = __builtin_fmaxf(-448.0f, __builtin_fminf(v[i] / scale, 448.0f));
  // the clamp leaves no NaN: the hardware conversion equals f32_to_e4m3 here
  const uint32_t w0 = e4m3x4_raw(y[0], y[1], y[2], y[3]), w1 = e4m3x4_raw(y[4], y[5], y[6], y[7]);
  if (!live) return;
  *reinterpret_cast<uint2*>(q + row * H + col * 128 + sub * 8) = make_uint2(w0, w1);
  if (sub == 0) scales[TRANSPOSED ? col * rows + row : row * (H / 128) + col] = scale;
}

// ------------------------------------------ residual + RMSNorm -> MXFP8

// Residual add + Gemma RMSNorm, then MXFP8 (or bf16) of the normalized row
// (mxfp6/mxfp8_norm_quant.py:15-39, mxfp6/gemma_norm.py:13-29).  One
// workgroup of 256 threads per row of N (N % 32 == 0, N <= 16384): thread t
// owns the 8-element chunks c = t, t + 256, ..., kept in registers between
// the two passes.  The variance is summed in a fixed order -- serially per
// thread, then lane 0 of an xor butterfly per wavefront, then the four
// wavefronts in order -- so the codes are a pure function of the input.  A
// 32-element block is four consecutive chunks held by four consecutive lanes
// of one iteration (N / 8 is a multiple of 4, so a quad is live or dead as a
// whole), quantized by quant8x4.
constexpr int kNormMaxChunks = 8;

template <bool QUANT, int RULE, bool SWIZZLED, bool RES>
__global__ __launch_bounds__(256) void rmsnorm_mx_kernel(const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ res,
                                                         const uint16_t* __restrict__ weight, int64_t N,
                                                         float eps, uint8_t* __restrict__ codes,
                                                         uint8_t* __restrict__ scales,
                                                         uint16_t* __restrict__ summed,
                                                         uint16_t* __restrict__ y) {
  __shared__ float wsum[4];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int64_t row = blockIdx.x;
  const int64_t chunks = N / 8;
  float v[kNormMaxChunks][8];
  float part = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormMaxChunks; ++i) {
    const int64_t c = t + 256 * i;
#pragma unroll
    for (int k = 0; k < 8; ++k) v[i][k] = 0.0f;
    if (c < chunks) {
      bf16x8_to_f32(*reinterpret_cast<const uint4*>(x + row * N + c * 8), v[i]);
      if (RES) {
        float r8[8];
        bf16x8_to_f32(*reinterpret_cast<const uint4*>(res + row * N + c * 8), r8);
#pragma unroll
        for (int k = 0; k < 8; ++k) v[i][k] = v[i][k] + r8[k];
        uint32_t h[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) h[k] = f32_to_bf16(v[i][2 * k]) | (uint32_t)f32_to_bf16(v[i][2 * k + 1]) << 16;
        *reinterpret_cast<uint4*>(summed + row * N + c * 8) = uint4{h[0], h[1], h[2], h[3]};
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) part = part + v[i][k] * v[i][k];
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) part = part + __shfl_xor(part, off);
  if (lane == 0) wsum[wv] = part;
  __syncthreads();
  const float total = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
  const float rs = 1.0f / __builtin_sqrtf(total / (float)N + eps);
#pragma unroll
  for (int i = 0; i < kNormMaxChunks; ++i) {
    if (256 * i >= chunks) break;  // uniform
    const int64_t c = t + 256 * i;
    const bool live = c < chunks;
    float w8[8], yv[8];
    bf16x8_to_f32(*reinterpret_cast<const uint4*>(weight + (live ? c : 0) * 8), w8);
#pragma unroll
    for (int k = 0; k < 8; ++k) yv[k] = bf16_round((v[i][k] * rs) * (w8[k] + 1.0f));
    if (QUANT) {
      uint32_t packed[2];
      const uint32_t sc = quant8x4<RULE>(yv, packed);
      if (!live) continue;
      *reinterpret_cast<uint2*>(codes + row * N + c * 8) = make_uint2(packed[0], packed[1]);
      if ((t & 3) == 0) {
        const int64_t blk = c / 4;
        if (SWIZZLED) scales[swizzle_offset(row, blk, N)] = (uint8_t)sc;
        else scales[row * (N / 32) + blk] = (uint8_t)sc;
      }
    } else if (live) {
      uint32_t h[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) h[k] = f32_to_bf16(yv[2 * k]) | (uint32_t)f32_to_bf16(yv[2 * k + 1]) << 16;
      *reinterpret_cast<uint4*>(y + row * N + c * 8) = uint4{h[0], h[1], h[2], h[3]};
    }
  }
}

}  // namespace mxl

// ------------------------------------------------------------------- C ABI

using namespace mxl;

static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// the kernels index lanes in 32 bits (BlockLane)
static inline bool lanes_fit(int64_t lanes) { return lanes <= (int64_t)0x7FFFFF00; }

extern "C" int mxl_quantize_mxfp8(const void* x, int64_t M, int64_t K, int64_t ldx, int rule,
                                  void* codes, void* scales, void* stream) {
  MXL_CHECK_ARG(M >= 0 && K > 0 && K % 32 == 0, "mxl_quantize_mxfp8: need K > 0, K %% 32 == 0 (K=%lld)", (long long)K);
  MXL_CHECK_ARG(ldx >= K && ldx % 8 == 0, "mxl_quantize_mxfp8: ldx must be >= K and a multiple of 8");
  MXL_CHECK_ARG(rule == kFloorCarry175 || rule == kCeilDiv448 || rule == kRpUe8m0, "mxl_quantize_mxfp8: unknown rule %d", rule);
  MXL_CHECK_ARG(aligned16(x) && aligned16(codes), "mxl_quantize_mxfp8: x and codes must be 16-byte aligned");
  MXL_CHECK_ARG(lanes_fit(M * (K / 32) * 4), "mxl_quantize_mxfp8: too large (M=%lld, K=%lld)", (long long)M, (long long)K);
  if (M == 0) return MXL_OK;
  const int64_t n = M * (K / 32) * 4;
  dim3 grid((unsigned)((n + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  if (rule == kFloorCarry175)
    quant_mxfp8_kernel<kFloorCarry175><<<grid, 256, 0, s>>>((const uint16_t*)x, ldx, (uint8_t*)codes, (uint8_t*)scales, M, K);
  else if (rule == kCeilDiv448)
    quant_mxfp8_kernel<kCeilDiv448><<<grid, 256, 0, s>>>((const uint16_t*)x, ldx, (uint8_t*)codes, (uint8_t*)scales, M, K);
  else
    quant_mxfp8_kernel<kRpUe8m0><<<grid, 256, 0, s>>>((const uint16_t*)x, ldx, (uint8_t*)codes, (uint8_t*)scales, M, K);
  MXL_CHECK_LAUNCH("mxl_quantize_mxfp8");
  return MXL_OK;
}

extern "C" int64_t mxl_swizzled_scale_bytes(int64_t M, int64_t K);

extern "C" int mxl_quantize_mxfp8_swizzled(const void* x, int64_t M, int64_t K, int64_t ldx, int rule, void* codes,
                                           void* scales, void* stream) {
  MXL_CHECK_ARG(M >= 0 && K > 0 && K % 32 == 0, "mxl_quantize_mxfp8_swizzled: need K > 0, K %% 32 == 0 (K=%lld)",
                (long long)K);
  MXL_CHECK_ARG(ldx >= K && ldx % 8 == 0, "mxl_quantize_mxfp8_swizzled: ldx must be >= K and a multiple of 8");
  MXL_CHECK_ARG(rule == kFloorCarry175 || rule == kCeilDiv448 || rule == kRpUe8m0,
                "mxl_quantize_mxfp8_swizzled: unknown rule %d", rule);
  MXL_CHECK_ARG(aligned16(x) && aligned16(codes), "mxl_quantize_mxfp8_swizzled: x and codes must be 16-byte aligned");
  MXL_CHECK_ARG(lanes_fit(M * (K / 32) * 4), "mxl_quantize_mxfp8_swizzled: too large (M=%lld, K=%lld)", (long long)M,
                (long long)K);
  if (M == 0) return MXL_OK;
  hipStream_t s = (hipStream_t)stream;
  uint8_t* sc = (uint8_t*)scales;
  if (M % 128 || (K / 32) % 4) {  // the layout has padding bytes: zero them
    const int64_t total = mxl_swizzled_scale_bytes(M, K);
    swizzle_pad_kernel<<<dim3((unsigned)((total + 255) / 256)), 256, 0, s>>>(sc, M, K, total);
  }
  const int64_t n = M * (K / 32) * 4;
  dim3 grid((unsigned)((n + 255) / 256));
  const uint16_t* in = (const uint16_t*)x;
  uint8_t* c = (uint8_t*)codes;
  if (rule == kFloorCarry175) quant_mxfp8_kernel<kFloorCarry175, true><<<grid, 256, 0, s>>>(in, ldx, c, sc, M, K);
  else if (rule == kCeilDiv448) quant_mxfp8_kernel<kCeilDiv448, true><<<grid, 256, 0, s>>>(in, ldx, c, sc, M, K);
  else quant_mxfp8_kernel<kRpUe8m0, true><<<grid, 256, 0, s>>>(in, ldx, c, sc, M, K);
  MXL_CHECK_LAUNCH("mxl_quantize_mxfp8_swizzled");
  return MXL_OK;
}

extern "C" int mxl_quantize_mxfp6(const void* x, int64_t M, int64_t K, int64_t ldx, int fmt, void* packed,
                                  void* scales, void* stream) {
  MXL_CHECK_ARG(M >= 0 && K > 0 && K % 32 == 0, "mxl_quantize_mxfp6: need K > 0, K %% 32 == 0 (K=%lld)", (long long)K);
  MXL_CHECK_ARG(fmt == kE2M3 || fmt == kE3M2, "mxl_quantize_mxfp6: fmt must be 2 (E2M3) or 3 (E3M2), got %d", fmt);
  MXL_CHECK_ARG(ldx >= K && ldx % 8 == 0, "mxl_quantize_mxfp6: ldx must be >= K and a multiple of 8");
  MXL_CHECK_ARG(aligned16(x) && ((uintptr_t)packed & 1) == 0, "mxl_quantize_mxfp6: misaligned buffers");
  MXL_CHECK_ARG(lanes_fit(M * (K / 32) * 4), "mxl_quantize_mxfp6: too large (M=%lld, K=%lld)", (long long)M, (long long)K);
  if (M == 0) return MXL_OK;
  const int64_t n = M * (K / 32) * 4;
  dim3 grid((unsigned)((n + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  if (fmt == kE2M3)
    quant_mxfp6_kernel<kE2M3><<<grid, 256, 0, s>>>((const uint16_t*)x, ldx, (uint8_t*)packed, (uint8_t*)scales, M, K);
  else
    quant_mxfp6_kernel<kE3M2><<<grid, 256, 0, s>>>((const uint16_t*)x, ldx, (uint8_t*)packed, (uint8_t*)scales, M, K);
  MXL_CHECK_LAUNCH("mxl_quantize_mxfp6");
  return MXL_OK;
}

extern "C" int mxl_quantize_mxfp8_dual(const void* x, int64_t M, int64_t K, int64_t ldx, int rule, void* hi,
                                       void* s_hi, void* res, void* s_res, void* stream) {
  MXL_CHECK_ARG(M >= 0 && K > 0 && K % 32 == 0 && ldx >= K && ldx % 8 == 0,
                "mxl_quantize_mxfp8_dual: need K %% 32 == 0, ldx >= K, ldx %% 8 == 0");
  MXL_CHECK_ARG(rule == kFloorCarry175 || rule == kCeilDiv448 || rule == kRpUe8m0, "mxl_quantize_mxfp8_dual: unknown rule %d", rule);
  MXL_CHECK_ARG(aligned16(x) && ((uintptr_t)hi & 7) == 0 && ((uintptr_t)res & 7) == 0,
                "mxl_quantize_mxfp8_dual: misaligned buffers");
  MXL_CHECK_ARG(lanes_fit(M * (K / 32) * 4), "mxl_quantize_mxfp8_dual: too large (M=%lld, K=%lld)", (long long)M, (long long)K);
  if (M == 0) return MXL_OK;
  const int64_t n = M * (K / 32) * 4;
  dim3 grid((unsigned)((n + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  if (rule == kFloorCarry175)
    quant_mxfp8_dual_kernel<kFloorCarry175><<<grid, 256, 0, s>>>((const uint16_t*)x, ldx, (uint8_t*)hi,
                                                                (uint8_t*)s_hi, (uint8_t*)res, (uint8_t*)s_res, M, K);
  else if (rule == kCeilDiv448)
    quant_mxfp8_dual_kernel<kCeilDiv448><<<grid, 256, 0, s>>>((const uint16_t*)x, ldx, (uint8_t*)hi,
                                                             (uint8_t*)s_hi, (uint8_t*)res, (uint8_t*)s_res, M, K);
  else
    quant_mxfp8_dual_kernel<kRpUe8m0><<<grid, 256, 0, s>>>((const uint16_t*)x, ldx, (uint8_t*)hi,
                                                          (uint8_t*)s_hi, (uint8_t*)res, (uint8_t*)s_res, M, K);
  MXL_CHECK_LAUNCH("mxl_quantize_mxfp8_dual");
  return MXL_OK;
}

extern "C" int64_t mxl_swizzled_scale_bytes(int64_t M, int64_t K) {
  return (M + 127) / 128 * 128 * ((K / 32 + 3) / 4) * 4;
}

extern "C" int mxl_swizzle_scales(const void* logical, int64_t R, int64_t K, void* swizzled, void* stream) {
  MXL_CHECK_ARG(R >= 0 && K > 0 && K % 32 == 0, "mxl_swizzle_scales: need K > 0, K %% 32 == 0 (K=%lld)", (long long)K);
  if (R == 0) return MXL_OK;
  const int64_t total = mxl_swizzled_scale_bytes(R, K);
  swizzle_scales_kernel<<<dim3((unsigned)((total + 255) / 256)), 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)logical, (uint8_t*)swizzled, R, K, total);
  MXL_CHECK_LAUNCH("mxl_swizzle_scales");
  return MXL_OK;
}

namespace {
template <bool SWIZZLED>
void launch_swiglu(int rule, bool table, dim3 grid, int threads, hipStream_t s, const uint16_t* in, uint8_t* c,
                   uint8_t* sc, int64_t M, int64_t K) {
  if (table && rule == kFloorCarry175)
    swiglu_mxfp8_kernel<kFloorCarry175, SWIZZLED, true><<<grid, threads, 0, s>>>(in, c, sc, M, K);
  else if (table)
    swiglu_mxfp8_kernel<kCeilDiv448, SWIZZLED, true><<<grid, threads, 0, s>>>(in, c, sc, M, K);
  else if (rule == kFloorCarry175)
    swiglu_mxfp8_kernel<kFloorCarry175, SWIZZLED, false><<<grid, threads, 0, s>>>(in, c, sc, M, K);
  else if (rule == kCeilDiv448)
    swiglu_mxfp8_kernel<kCeilDiv448, SWIZZLED, false><<<grid, threads, 0, s>>>(in, c, sc, M, K);
  else
    swiglu_mxfp8_kernel<kRpUe8m0, SWIZZLED, false><<<grid, threads, 0, s>>>(in, c, sc, M, K);
}
}  // namespace

extern "C" int mxl_swiglu_mxfp8(const void* gate_up, int64_t M, int64_t K, int rule, int swizzled,
                                void* codes, void* scales, void* stream) {
  MXL_CHECK_ARG(M >= 0 && K > 0 && K % 32 == 0, "mxl_swiglu_mxfp8: need K > 0, K %% 32 == 0 (K=%lld)", (long long)K);
  MXL_CHECK_ARG(rule == kFloorCarry175 || rule == kCeilDiv448 || rule == kRpUe8m0, "mxl_swiglu_mxfp8: unknown rule %d", rule);
  MXL_CHECK_ARG(aligned16(gate_up) && aligned16(codes), "mxl_swiglu_mxfp8: gate_up and codes must be 16-byte aligned");
  MXL_CHECK_ARG(lanes_fit(M * (K / 32) * 4), "mxl_swiglu_mxfp8: too large (M=%lld, K=%lld)", (long long)M, (long long)K);
  if (M == 0) return MXL_OK;
  const int64_t n = M * (K / 32) * 4;
  // with the table at most two workgroups per CU (each stages the 16 KiB table once),
  // striding over the items
  const bool table = rule != kRpUe8m0 && n >= kSwigluTableItemsPerCu * cu_count();
  const int threads = table ? kSwigluThreads : 256;
  dim3 grid((unsigned)(table ? std::min<int64_t>((n + threads - 1) / threads, 2 * (int64_t)cu_count())
                             : (n + threads - 1) / threads));
  hipStream_t s = (hipStream_t)stream;
  const uint16_t* in = (const uint16_t*)gate_up;
  uint8_t* c = (uint8_t*)codes;
  uint8_t* sc = (uint8_t*)scales;
  if (swizzled) {
    if (M % 128 || (K / 32) % 4) {  // the layout has padding bytes: zero them
      const int64_t total = mxl_swizzled_scale_bytes(M, K);
      swizzle_pad_kernel<<<dim3((unsigned)((total + 255) / 256)), 256, 0, s>>>(sc, M, K, total);
    }
    launch_swiglu<true>(rule, table, grid, threads, s, in, c, sc, M, K);
  } else {
    launch_swiglu<false>(rule, table, grid, threads, s, in, c, sc, M, K);
  }
  MXL_CHECK_LAUNCH("mxl_swiglu_mxfp8");
  return MXL_OK;
}

extern "C" int mxl_quantize_block_fp8(const void* x, int64_t M, int64_t K, void* q, void* s_colmajor,
                                      void* stream) {
  MXL_CHECK_ARG(M >= 0 && K > 0 && K % 128 == 0, "mxl_quantize_block_fp8: need K %% 128 == 0 (K=%lld)", (long long)K);
  MXL_CHECK_ARG(aligned16(x) && ((uintptr_t)q & 7) == 0, "mxl_quantize_block_fp8: misaligned buffers");
  MXL_CHECK_ARG(lanes_fit(M * (K / 128) * 16), "mxl_quantize_block_fp8: too large (M=%lld, K=%lld)", (long long)M, (long long)K);
  if (M == 0) return MXL_OK;
  const int64_t threads = M * (K / 128) * 16;
  quant_block_fp8_kernel<<<dim3((unsigned)((threads + 255) / 256)), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)x, (uint8_t*)q, (float*)s_colmajor, M, K);
  MXL_CHECK_LAUNCH("mxl_quantize_block_fp8");
  return MXL_OK;
}

extern "C" int mxl_silu_mul_block_fp8(const void* input, int64_t rows, int64_t H, int transposed, void* q,
                                      void* scales, void* stream) {
  MXL_CHECK_ARG(rows >= 0 && H > 0 && H % 128 == 0, "mxl_silu_mul_block_fp8: need H %% 128 == 0 (H=%lld)", (long long)H);
  MXL_CHECK_ARG(aligned16(input) && ((uintptr_t)q & 7) == 0, "mxl_silu_mul_block_fp8: misaligned buffers");
  MXL_CHECK_ARG(lanes_fit(rows * (H / 128) * 16), "mxl_silu_mul_block_fp8: too large (rows=%lld, H=%lld)", (long long)rows, (long long)H);
  if (rows == 0) return MXL_OK;
  const int64_t threads = rows * (H / 128) * 16;
  dim3 grid((unsigned)((threads + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  if (transposed)
    silu_mul_block_fp8_kernel<true><<<grid, 256, 0, s>>>((const uint16_t*)input, (uint8_t*)q, (float*)scales, rows, H);
  else
    silu_mul_block_fp8_kernel<false><<<grid, 256, 0, s>>>((const uint16_t*)input, (uint8_t*)q, (float*)scales, rows, H);
  MXL_CHECK_LAUNCH("mxl_silu_mul_block_fp8");
  return MXL_OK;
}

namespace {
template <bool QUANT, int RULE, bool SWZ>
void launch_rmsnorm(const void* x, const void* residual, const void* weight, int64_t M, int64_t N, float eps,
                    void* codes, void* scales, void* summed, void* y, hipStream_t s) {
  const dim3 grid((unsigned)M);
  if (residual)
    mxl::rmsnorm_mx_kernel<QUANT, RULE, SWZ, true><<<grid, 256, 0, s>>>(
        (const uint16_t*)x, (const uint16_t*)residual, (const uint16_t*)weight, N, eps, (uint8_t*)codes,
        (uint8_t*)scales, (uint16_t*)summed, (uint16_t*)y);
  else
    mxl::rmsnorm_mx_kernel<QUANT, RULE, SWZ, false><<<grid, 256, 0, s>>>(
        (const uint16_t*)x, nullptr, (const uint16_t*)weight, N, eps, (uint8_t*)codes, (uint8_t*)scales,
        nullptr, (uint16_t*)y);
}

int check_norm_args(const char* what, const void* x, const void* residual, const void* weight, int64_t M, int64_t N,
                    const void* summed) {
  MXL_CHECK_ARG(M >= 0 && N >= 32 && N % 32 == 0 && N <= 256 * 8 * mxl::kNormMaxChunks,
                "%s: need 32 <= N <= %d, N %% 32 == 0 (N=%lld)", what, 256 * 8 * mxl::kNormMaxChunks, (long long)N);
  MXL_CHECK_ARG(M <= 0x7FFFFFFF, "%s: too many rows (%lld)", what, (long long)M);
  MXL_CHECK_ARG(aligned16(x) && aligned16(weight) && (!residual || aligned16(residual)),
                "%s: x, residual and weight must be 16-byte aligned", what);
  MXL_CHECK_ARG(!residual || (summed && aligned16(summed)), "%s: a residual needs a 16-byte aligned summed output",
                what);
  return MXL_OK;
}
}  // namespace

extern "C" int mxl_rmsnorm_mxfp8(const void* x, const void* residual, const void* weight, int64_t M, int64_t N,
                                 float eps, int rule, int swizzled, void* codes, void* scales, void* summed,
                                 void* stream) {
  int rc = check_norm_args("mxl_rmsnorm_mxfp8", x, residual, weight, M, N, summed);
  if (rc != MXL_OK) return rc;
  MXL_CHECK_ARG(rule == kFloorCarry175 || rule == kCeilDiv448, "mxl_rmsnorm_mxfp8: unknown rule %d", rule);
  MXL_CHECK_ARG(((uintptr_t)codes & 7) == 0, "mxl_rmsnorm_mxfp8: codes must be 8-byte aligned");
  if (M == 0) return MXL_OK;
  hipStream_t s = (hipStream_t)stream;
  if (swizzled) {
    const int64_t total = mxl_swizzled_scale_bytes(M, N);
    mxl::swizzle_pad_kernel<<<dim3((unsigned)((total + 255) / 256)), 256, 0, s>>>((uint8_t*)scales, M, N, total);
    if (rule == kFloorCarry175) launch_rmsnorm<true, kFloorCarry175, true>(x, residual, weight, M, N, eps, codes, scales, summed, nullptr, s);
    else launch_rmsnorm<true, kCeilDiv448, true>(x, residual, weight, M, N, eps, codes, scales, summed, nullptr, s);
  } else {
    if (rule == kFloorCarry175) launch_rmsnorm<true, kFloorCarry175, false>(x, residual, weight, M, N, eps, codes, scales, summed, nullptr, s);
    else launch_rmsnorm<true, kCeilDiv448, false>(x, residual, weight, M, N, eps, codes, scales, summed, nullptr, s);
  }
  MXL_CHECK_LAUNCH("mxl_rmsnorm_mxfp8");
  return MXL_OK;
}

extern "C" int mxl_gemma_rmsnorm(const void* x, const void* residual, const void* weight, int64_t M, int64_t N,
                                 float eps, void* y, void* summed, void* stream) {
  int rc = check_norm_args("mxl_gemma_rmsnorm", x, residual, weight, M, N, summed);
  if (rc != MXL_OK) return rc;
  MXL_CHECK_ARG(aligned16(y), "mxl_gemma_rmsnorm: y must be 16-byte aligned");
  if (M == 0) return MXL_OK;
  launch_rmsnorm<false, kCeilDiv448, false>(x, residual, weight, M, N, eps, nullptr, nullptr, summed, y,
                                            (hipStream_t)stream);
  MXL_CHECK_LAUNCH("mxl_gemma_rmsnorm");
  return MXL_OK;
}
