// Declarations shared by the GEMM kernels (gemm.hip, gemm_wide.hip, gemm_stream.hip).
#pragma once

#include "mx_common.h"

namespace mxl {

constexpr int kTileK = 512;

template <int FMT>
struct FmtTraits;
template <>
struct FmtTraits<kE4M3> { static constexpr int CH = 8; static constexpr int RUN = 32; };
template <>
struct FmtTraits<kE2M3> { static constexpr int CH = 6; static constexpr int RUN = 24; };
template <>
struct FmtTraits<kE3M2> { static constexpr int CH = 6; static constexpr int RUN = 24; };

__host__ __device__ inline int tile_chunks(int fmt) { return fmt == kE4M3 ? 8 : 6; }

struct GemmParams {
  const uint8_t* a;      // activation codes, row-major
  const void* sa;        // MX: E8M0 [rows, K/32]; block-FP8: fp32 column-major [K/128, M]
  const uint8_t* w;      // tiled weight codes (expert 0)
  const void* sw;        // MX: tiled scales; block-FP8: fp32 [ceil(N/128), K/128]
  const uint16_t* bias;  // bf16 [N] or null
  uint16_t* out;         // bf16, row stride ldc
  float* partial;        // [S, rows, N] when split
  const uint8_t* a2;     // two-limb activations: residual codes (gemm_kernel only), or null
  const void* sa2;       // and their E8M0 scales
  const int32_t* row_index;     // grouped: sorted_routes (A row = row_index[r] / row_div)
  const int64_t* expert_offsets;
  int64_t lda, ldc, M, N, K, KT, a_rows;
  int64_t w_expert_stride, sw_expert_stride;
  int row_div, S;
  int sa_swz = 0;     // MX activation scales: 0 logical [rows, K/32], 1 swizzled 128 x 4 tiles
  int64_t sa_ss = 4;  // bytes between the scale dwords of consecutive K128 slices of a row (4 or 512)
  float alpha = 1.0f;  // output scale, applied to the fp32 sum before its one rounding
  int out_f16 = 0;     // output element format: 0 bf16, 1 fp16
  // Grouped down projection with the weighted combine (gemm_stream_grouped_kernel,
  // COMB): routed output row p belongs to route comb_routes[p] = t * comb_topk + k; the
  // token rows are summed into comb_out [comb_T, N] bf16 by the unit that stores a
  // token's last row (comb_cnt: one zeroed int32 counter per token, left zero).
  uint16_t* comb_out = nullptr;
  const float* comb_w = nullptr;         // fp32 [comb_T, comb_topk] route weights
  const int32_t* comb_inv = nullptr;     // [comb_T * comb_topk] routed row of route (t, k), -1 dropped
  const int32_t* comb_routes = nullptr;  // [routed rows] route of each routed row
  int32_t* comb_cnt = nullptr;
  int64_t comb_T = 0;
  int comb_topk = 0;
  // Weight-streaming GEMM with its activation producer in the same launch (M <= 16,
  // gemm_stream_kernel FPROD): the bf16 input (gate/up [M, 2K] or x [M, K], row stride
  // fsrc_ld) is produced into p.a / p.sa, a per-stream slot of the library's scratch;
  // fsync: the slot's grid handoff counters (arrive, depart), zero between launches.
  const uint16_t* fsrc = nullptr;
  int64_t fsrc_ld = 0;
  uint32_t* fsync = nullptr;
};

// Output element formats (mxl_gemm_options.out_dtype).
enum OutFmt : int { kOutBf16 = 0, kOutF16 = 1 };

// round-to-nearest-even binary32 -> binary16 (v_cvt_f16_f32: overflow to infinity,
// subnormal results kept), NaN -> 0x7E00
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return f != f ? (uint16_t)0x7E00 : __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// The bits of one output element from its fp32 sum v: alpha v rounded once to the output
// format; with a bias (bf16 bits, `has_bias`) the rounded value plus the bias in binary32,
// rounded again (y + bias in the output format).  alpha = 1 leaves v unchanged, so a bf16
// output without scaling is f32_to_bf16(v).
__device__ __forceinline__ uint16_t out_bits(float v, float alpha, int f16, bool has_bias, uint16_t bias) {
  const float y = v * alpha;
  if (!f16) {
    const uint16_t h = f32_to_bf16(y);
    return has_bias ? f32_to_bf16(bf16_to_f32(h) + bf16_to_f32(bias)) : h;
  }
  const uint16_t h = f32_to_f16(y);
  return has_bias ? f32_to_f16(f16_to_f32(h) + bf16_to_f32(bias)) : h;
}
__device__ __forceinline__ uint16_t out_bits(const GemmParams& p, float v, int64_t col) {
  return out_bits(v, p.alpha, p.out_f16, p.bias != nullptr, p.bias ? p.bias[col] : (uint16_t)0);
}

// Byte offset of row `row`'s scale dword of K128 slice 0; slice s is sa_ss bytes further.
// Logical: row * K/32.  Swizzled (the reference's activation layout, 128-row x 4-group
// tiles of 512 bytes, groups padded to a multiple of 4): byte (r, g) sits at
// (((r / 128) T + g / 4) 32 + r % 32) 16 + ((r % 128) / 32) 4 + g % 4, T = ceil(K / 128).
__host__ __device__ inline int64_t sa_row_offset(const GemmParams& p, int64_t row) {
  if (!p.sa_swz) return row * (p.K / 32);
  const int64_t T = (p.K / 32 + 3) / 4;
  return (row >> 7) * T * 512 + (row & 31) * 16 + ((row & 127) >> 5) * 4;
}

// Byte offset, from a row's slice-0 scale dword, of the dword of the K128 slice holding
// K index ks (clamped to the last slice).  32-bit arithmetic: the slice count and the
// stride (4 or 512) keep the product far below 2^32, and the narrower math keeps the
// decode kernels inside their register budgets.
__host__ __device__ inline uint32_t scale_slice_offset(const GemmParams& p, int64_t ks) {
  return (uint32_t)((ks < p.K ? ks : p.K - 128) >> 7) * (uint32_t)p.sa_ss;
}

inline void set_sa_layout(GemmParams& p, int swizzled) {
  p.sa_swz = swizzled ? 1 : 0;
  p.sa_ss = swizzled ? 512 : 4;
}

// Sum of S fp32 split partials of 8 consecutive columns (split k at src + k * stride,
// 16-byte aligned), added in split order starting from split 0 itself.  The loads of
// up to eight splits are issued before their adds, so a thread waits on memory once
// per eight splits instead of once per split.
__device__ __forceinline__ void sum_splits8(const float* src, int64_t stride, int S, float4& lo, float4& hi) {
  lo = *reinterpret_cast<const float4*>(src);
  hi = *reinterpret_cast<const float4*>(src + 4);
  for (int k0 = 1; k0 < S; k0 += 8) {
    float4 a[8], b[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (k0 + u < S) {
        const float* p = src + (int64_t)(k0 + u) * stride;
        a[u] = *reinterpret_cast<const float4*>(p);
        b[u] = *reinterpret_cast<const float4*>(p + 4);
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (k0 + u < S) {
        lo.x += a[u].x; lo.y += a[u].y; lo.z += a[u].z; lo.w += a[u].w;
        hi.x += b[u].x; hi.y += b[u].y; hi.z += b[u].z; hi.w += b[u].w;
      }
    }
  }
}

// Per-call selection: the scale layout of A and the tuning overrides (the reference's
// tactic / splits overrides, src/vllm_mach/mxfp8/native_backend.py:29).  Same layout
// as mxl_gemm_options in include/mxlinear.h.
enum KernelChoice : int { kAuto = -1, kStream = 0, kWide = 1, kGeneric = 2, kStreamWide = 3, kChunk = 4 };
struct GemmOptions {
  int sa_layout = 0;  // 0 logical, 1 swizzled
  int kernel = kAuto;
  int splits = 0;     // 0: the cost model's; else the K split (wide, generic)
  int tile_n = 0;     // wide: NT in {1, 2, 4}; 0 auto
  int tile_m = 0;     // wide: MT in {4, 8}; 0 auto
  int hybrid = 0;     // wide, splits == 1: full rounds whole-K, the remainder split
  int waves = 0;      // wide MX dense, 128-row tiles: 4 or 8 waves per workgroup; 0 auto
  int out_dtype = kOutBf16;  // output element format
  float alpha = 1.0f;        // output scale
};

template <int MT>
struct ATile {
  v8i d[MT][4];
  uint32_t s[MT][4];  // MX: raw scale dword of MFMA j; the lane uses byte q (extracted at use)
};

// Load the activation operands of one super-tile for MT 16-row tiles.  A
// super-tile wholly inside K takes a branch-free path (a uniform condition),
// so the loads are not waited on before the MFMAs that consume them.
// The loads are row-major: `arow[mt]` is the row this lane reads, row lane / 4
// of m-tile mt, piece lane % 4, so four neighbouring lanes move one row's 64
// bytes in one access (lanes on sixteen rows, the fragment order, would cost an
// access each); a lane-permute then hands fragment lane 16 q + r its piece q of
// row r.
template <int MT, bool BLOCK>
__device__ __forceinline__ void load_a(const GemmParams& p, const int64_t (&arow)[MT], int64_t kt, int lane,
                                       ATile<MT>& t) {
  const bool full = (kt + 1) * kTileK <= p.K;
  const int cp = lane & 3, r = lane & 15, q = lane >> 4;
  const int from = 4 * (4 * r + q);  // byte address of the source lane 4 r + q
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const uint8_t* base = p.a + arow[mt] * p.lda;
    const uint8_t* sbase = static_cast<const uint8_t*>(p.sa) + (BLOCK ? 0 : sa_row_offset(p, arow[mt]));
    uint32_t sd = 0;
    if (!BLOCK) {  // scale dword of slice cp (clamped inside K; slices past K are zeroed below)
      const int64_t ks = kt * kTileK + 128 * cp;
      sd = *reinterpret_cast<const uint32_t*>(sbase + scale_slice_offset(p, ks));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t k0 = kt * kTileK + 128 * j;
      if (full || k0 < p.K) {
        const uint4 lo = *reinterpret_cast<const uint4*>(base + k0 + 16 * cp);
        const uint4 hi = *reinterpret_cast<const uint4*>(base + k0 + 64 + 16 * cp);
        const uint32_t x[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        int y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = __builtin_amdgcn_ds_bpermute(from, (int)x[e]);
        t.d[mt][j] = v8i{y[0], y[1], y[2], y[3], y[4], y[5], y[6], y[7]};
        t.s[mt][j] = BLOCK ? 0u : (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (4 * r + j), (int)sd);
      } else {
        t.d[mt][j] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
        t.s[mt][j] = 0;
      }
    }
  }
}

template <int FMT, int NT>
struct BTile {
  uint4 c[NT][FmtTraits<FMT>::CH];
  uint32_t s[NT];
};

template <int FMT>
__device__ __forceinline__ v8i b_operand(const uint4* c, int j) {
  if (FMT == kE4M3) {
    const uint4 lo = c[2 * j], hi = c[2 * j + 1];
    return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  } else {
    // the lane's 24 dwords; MFMA j takes dwords [6j, 6j + 6)
    uint32_t d[24];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      d[4 * i] = c[i].x; d[4 * i + 1] = c[i].y; d[4 * i + 2] = c[i].z; d[4 * i + 3] = c[i].w;
    }
    return v8i{(int)d[6 * j], (int)d[6 * j + 1], (int)d[6 * j + 2], (int)d[6 * j + 3],
               (int)d[6 * j + 4], (int)d[6 * j + 5], 0, 0};
  }
}

template <int FMT, int NT, bool BLOCK>
__device__ __forceinline__ void load_b(const GemmParams& p, const uint8_t* w, const uint8_t* sw,
                                       const int64_t (&ntile)[NT], int64_t kt, int lane, BTile<FMT, NT>& t) {
  constexpr int CH = FmtTraits<FMT>::CH;
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const uint8_t* base = w + (ntile[n] * p.KT + kt) * (CH * 1024) + lane * 16;
#pragma unroll
    for (int c = 0; c < CH; ++c) t.c[n][c] = *reinterpret_cast<const uint4*>(base + c * 1024);
    if (!BLOCK) t.s[n] = *reinterpret_cast<const uint32_t*>(sw + (ntile[n] * p.KT + kt) * 256 + lane * 4);
  }
}

// The B-format and op_sel operands must be immediates.
template <int FMT, int J>
__device__ __forceinline__ v4f mfma_step(v8i a, v8i b, v4f c, uint32_t sa, uint32_t sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, kE4M3, FMT, 0, (int)sa, J, (int)sb);
}

// Both scale operands packed by slice: byte J of sa and of sb
template <int FMT, int J>
__device__ __forceinline__ v4f mfma_step_packed(v8i a, v8i b, v4f c, uint32_t sa, uint32_t sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, kE4M3, FMT, J, (int)sa, J, (int)sb);
}

template <int FMT>
__device__ __forceinline__ v4f mfma_raw(v8i a, v8i b) {
  const v4f z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, kE4M3, FMT, 0, 127, 0, 127);
}

// Wide-tile LDS-pipelined kernel for prefill-sized M (gemm_wide.hip): NT
// n-tiles per wave (workgroup tile 16 MT x 64 NT), S K-splits of kt_per_split
// 512-wide super-tiles each.  Hybrid (dp_tiles > 0, S = 1): the first dp_tiles
// output tiles run whole-K in full rounds of the CUs, the remaining ones split
// K S2 ways (kt2 super-tiles each) into compact partials summed by a tile reduce.
struct WideConfig {
  int NT, S;
  int64_t kt_per_split;
  int64_t dp_tiles = 0;
  int S2 = 1;
  int64_t kt2 = 0;
  int MT = 8;  // 16-row m-tiles per workgroup tile: 8 (128 rows) or 4 (64 rows)
  int WM = 1;  // m-groups of four waves: 1, or 2 (eight waves, each half the tile's rows)
};
// The cost model's choice, or the options' tile / split overrides where given.
WideConfig wide_config(int64_t M, int64_t N, int64_t K, int fmt, const GemmOptions& o = GemmOptions());
// Workspace bytes a configuration needs (split partials), 0 when none.
int64_t wide_workspace_bytes(const WideConfig& c, int64_t M, int64_t N);
bool wide_gemm_eligible(int64_t M, int64_t K);
// Grouped wide kernel: at most this many experts (their prefix lives in LDS).
constexpr int64_t kWideGroupedMaxExperts = 1024;
// Block-FP8 wide kernel: at most this many K128 stages per K split (each wave keeps
// its weight block scales of the split in LDS), so K <= 32768.
constexpr int kWideBlockStages = 256;
// m-tiles per unit of the grouped weight-streaming variant for tens of rows per expert
// (96 rows: one unit per expert at 64 rows per expert on average; with 80-row units the
// few experts past 80 rows made some CUs run two units, 107 against 74 us at c5)
constexpr int kGroupedStreamWideMT = 6;
int cu_count();
hipError_t launch_gemm_wide(int fmt, bool block, const WideConfig& c, const GemmParams& p, int64_t num_experts,
                            hipStream_t s);



// K-chunked weight-streaming kernel for up to 128 rows (gemm_chunk.hip), MX weights:
// chunks of kChunkSuperTiles super-tiles, fp32 partials [chunks][M][N] when K has more
// than one chunk; preferred by the planner only where it measured faster.
constexpr int kChunkSuperTiles = 4;
bool chunk_gemm_eligible(int64_t M, int64_t K, int fmt);
bool chunk_gemm_preferred(int64_t M, int64_t N, int64_t K);
int64_t chunk_count(int64_t K, int kc);
hipError_t launch_gemm_chunk(int fmt, const GemmParams& p, hipStream_t s);

// Weight-streaming kernel for decode-sized M (gemm_stream.hip), MX or block-FP8.
bool stream_gemm_eligible(int64_t M, int64_t K, bool block);
// Most K super-tiles the one-super-tile-per-wave variant takes (more: two per wave).
int stream_max_waves(bool block);
hipError_t launch_gemm_stream(int fmt, bool block, const GemmParams& p, hipStream_t s);
// One activation row computed from its bf16 gate/up row inside the weight-streaming
// GEMM (p.a = gate_up, M = 1, SwiGLU rule 1 or 2)
bool stream_swiglu_eligible(int64_t M, int64_t K, int rule);
hipError_t launch_gemm_stream_swiglu(int fmt, int rule, const GemmParams& p, hipStream_t s);
// One bf16 activation row (p.a, M = 1) quantized to MXFP8 inside the weight-streaming GEMM
// (the activation quantizer's arithmetic, rule 0, 1 or 2)
bool stream_quant_row_eligible(int64_t M, int64_t K, int rule);
hipError_t launch_gemm_stream_quant_row(int fmt, int rule, const GemmParams& p, hipStream_t s);
// MXFP8 quantization of up to 16 bf16 rows inside the weight-streaming GEMM, each fragment
// lane quantizing its own pieces (K <= 4096)
// One bf16 row block-FP8 quantized inside the block-FP8 weight-streaming GEMM by every
// wavefront (M = 1, the stream path's K range), bit-identical to the quantizer + GEMM.
bool stream_block_row_eligible(int64_t M, int64_t K);
hipError_t launch_gemm_stream_block_row(const GemmParams& p, hipStream_t s);
bool stream_quant_rows_eligible(int64_t M, int64_t K, int rule);
hipError_t launch_gemm_stream_quant_rows(int fmt, int rule, const GemmParams& p, hipStream_t s);
// Producer + weight-streaming GEMM in one launch (M <= 16): prod 1 / 2 = SwiGLU ->
// MXFP8 under that rule (p.fsrc = gate/up [M, 2K]), 4 + rule = the MXFP8 activation
// quantizer, kFusedBlockFp8 = the block-FP8 quantizer (p.fsrc = x [M, K]); p.fsrc_ld is
// the input's row stride.  Sets p.a / p.sa to the stream's scratch slot and launches;
// returns an MXL status (MXL_EUNSUPPORTED when the shape does not fit one launch).
constexpr int kFusedBlockFp8 = 8;
bool stream_fused_eligible(int64_t M, int64_t K, bool block, int fmt);
int launch_gemm_stream_fused(int fmt, int prod, GemmParams& p, hipStream_t s, const char* who);
// Grouped (MoE) variant: persistent workgroups over (expert, up to 16 mt rows) units,
// each streaming the expert's weights; mt = 1 (few rows per expert) or 8.
bool stream_grouped_eligible(int64_t K, int64_t num_experts, int fmt, int mt);
// With prod = 1 (MXFP8 quantization of gathered bf16 rows) or 2 (SwiGLU of bf16 gate/up
// rows then MXFP8) each workgroup produces its unit's operands into LDS itself, rule
// `rule`; p.a then holds the bf16 input.  The unit's produced operands must fit
// kGroupedStageMaxBytes of LDS beside the kernel's own.
constexpr int64_t kGroupedStageMaxBytes = 64 * 1024;
bool stream_grouped_fused_eligible(int64_t K, int64_t num_experts, int fmt, int mt);
hipError_t launch_gemm_stream_grouped(int fmt, const GemmParams& p, int64_t num_experts, int mt, hipStream_t s,
                                      int prod = 0, int rule = 0, bool combine = false);

}  // namespace mxl
