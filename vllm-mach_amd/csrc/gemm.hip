// Block-scaled GEMMs on CDNA4 scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4).
//
// y[m, n] = sum_k a[m, k] * w[n, k] with
//   MX (MXFP8 / MXFP6): a = E4M3 codes * 2^(sa - 127) per 32 along K,
//                       w = E4M3 | E2M3 | E3M2 codes * 2^(sw - 127) per 32;
//                       the E8M0 scales are applied inside the MFMA.
//   block-FP8:          a = E4M3 * sa[m, k/128] (fp32), w = E4M3 * sb[n/128, k/128];
//                       each K128 block is one unscaled MFMA whose fp32 result is
//                       folded into the accumulator with fma(raw, sa*sb, acc).
//
// Operand layout of the 16x16x128 scaled MFMA (measured on gfx950): lane
// l = 16q + r supplies row r of A (column r of B).  For 8-bit codes its 32
// bytes are K [16q, 16q+16) followed by K [64+16q, 64+16q+16); for FP6 its 32
// values (24 bytes, little-endian 6-bit fields) are K [32q, 32q+32).  The E8M0
// scale of K block b = [32b, 32b+32) is taken from lane group q = b (op_sel
// picks the byte).  C: lane l holds rows 4q + i, column r.
//
// Weights live in an MFMA-tiled layout written once at load time:
//   tile (nt, kt) = weight rows [16nt, 16nt+16) x K [512kt, 512kt+512)
//   CH 1 KiB chunks (CH = 8 for 8-bit codes, 6 for FP6); lane l's 16 bytes of
//   chunk c are at c*1024 + 16l, so one 16-byte load per lane moves 1 KiB of
//   contiguous memory per wavefront.  Lane l concatenates its operand bytes for
//   MFMA j = 0..3 (K [512kt + 128j, +128)): 32 bytes (E4M3) or 24 bytes (FP6).
//   The MX scale tile is 256 bytes: lane l's dword holds, in byte j, the E8M0
//   of block 16kt + 4j + q of row r, so the MFMA takes it with op_sel = j.
//   Tiles are ordered (nt, kt) with kt fastest, so a wave walking K streams one
//   contiguous region.
//
// Activations stay row-major (the producers' natural layout and the gather
// layout the MoE path needs).  MFMA j needs, at lane l, row r's two 16-byte
// pieces at K 512kt + 128j + 16q and + 64 and byte q of the E8M0 dword of
// block 16kt + 4j; the loads are issued row by row (four neighbouring lanes
// read one row's 64 bytes, which the memory pipeline serves as one access)
// and a lane permute delivers each lane its pieces.
//
// Work split: a workgroup of KW wavefronts owns an MT x NT grid of 16x16
// output tiles; its waves take interleaved 512-wide K super-tiles and their
// fp32 partials are summed in LDS in wave order.  When the tile grid alone
// cannot fill 256 CUs, S workgroups split K further and write fp32 partials
// that a second kernel sums in split order: both orders are fixed, so every
// result is deterministic.
#include <atomic>
#include <mutex>
#include <string>
#include <unordered_map>
#include <string.h>
#include <stdio.h>

#include "gemm_common.h"

namespace mxl {

// ------------------------------------------------------------ weight packing

// One thread writes one 16-byte (chunk, lane) piece of one tile.
__global__ void pack_weight_kernel(const uint8_t* __restrict__ src, int64_t ld_src, uint8_t* __restrict__ dst,
                                   int64_t N, int64_t K, int64_t KT, int CH, int fp6, int64_t total) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= total) return;
  const int lane = (int)(id & 63);
  const int64_t c = (id >> 6) % CH;
  const int64_t tile = (id >> 6) / CH;
  const int64_t nt = tile / KT, kt = tile - nt * KT;
  const int r = lane & 15, q = lane >> 4;
  const int64_t row = nt * 16 + r;
  uint8_t out[16];
  if (!fp6) {
    const int j = (int)(c >> 1), half = (int)(c & 1);
    const int64_t base = kt * kTileK + 128 * j;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row < N && base < K) v = *reinterpret_cast<const uint4*>(src + row * ld_src + base + 16 * q + 64 * half);
    *reinterpret_cast<uint4*>(dst + tile * (CH * 1024) + c * 1024 + lane * 16) = v;
    return;
  }
#pragma unroll
  for (int b = 0; b < 16; ++b) {
    const int cb = (int)c * 16 + b;          // byte within the lane's 96-byte run
    const int j = cb / 24, o = cb % 24;
    const int64_t k0 = kt * kTileK + 128 * j + 32 * q;
    uint8_t v = 0;
    if (row < N && k0 < K) v = src[row * ld_src + k0 * 3 / 4 + o];
    out[b] = v;
  }
  uint4 w;
  w.x = out[0] | (out[1] << 8) | (out[2] << 16) | ((uint32_t)out[3] << 24);
  w.y = out[4] | (out[5] << 8) | (out[6] << 16) | ((uint32_t)out[7] << 24);
  w.z = out[8] | (out[9] << 8) | (out[10] << 16) | ((uint32_t)out[11] << 24);
  w.w = out[12] | (out[13] << 8) | (out[14] << 16) | ((uint32_t)out[15] << 24);
  *reinterpret_cast<uint4*>(dst + tile * (CH * 1024) + c * 1024 + lane * 16) = w;
}

// One thread writes one lane's scale dword of one tile.  The source is the logical
// [N, K/32] layout, or (swizzled) the reference's 128-row x 4-group tiles.
__global__ void pack_scale_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t N,
                                  int64_t K, int64_t KT, int64_t total, int swizzled) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= total) return;
  const int lane = (int)(id & 63);
  const int64_t tile = id >> 6;
  const int64_t nt = tile / KT, kt = tile - nt * KT;
  const int r = lane & 15, q = lane >> 4;
  const int64_t row = nt * 16 + r;
  uint32_t w = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t blk = kt * 16 + 4 * j + q;
    if (row < N && blk * 32 < K) {
      const int64_t off = swizzled ? (((row >> 7) * ((K / 32 + 3) / 4) + (blk >> 2)) * 32 + (row & 31)) * 16 +
                                         ((row & 127) >> 5) * 4 + (blk & 3)
                                   : row * (K / 32) + blk;
      w |= (uint32_t)src[off] << (8 * j);
    }
  }
  *reinterpret_cast<uint32_t*>(dst + tile * 256 + lane * 4) = w;
}

// ------------------------------------------------------------- GEMM kernel

// Accumulate one super-tile into acc[MT][NT].
template <int FMT, int MT, int NT, bool BLOCK>
__device__ __forceinline__ void compute_tile(const GemmParams& p, const ATile<MT>& A, const BTile<FMT, NT>& B,
                                             v4f (&acc)[MT][NT], int64_t kt, int q, const int64_t (&r4)[MT],
                                             int64_t hi, const int64_t (&ntile)[NT], const float* sb_rows) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const v8i b = b_operand<FMT>(B.c[n], j);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (!BLOCK) {
          const uint32_t sb = B.s[n];
          const uint32_t sa = (A.s[mt][j] >> (8 * q)) & 0xFFu;
          if (j == 0) acc[mt][n] = mfma_step<FMT, 0>(A.d[mt][j], b, acc[mt][n], sa, sb);
          if (j == 1) acc[mt][n] = mfma_step<FMT, 1>(A.d[mt][j], b, acc[mt][n], sa, sb);
          if (j == 2) acc[mt][n] = mfma_step<FMT, 2>(A.d[mt][j], b, acc[mt][n], sa, sb);
          if (j == 3) acc[mt][n] = mfma_step<FMT, 3>(A.d[mt][j], b, acc[mt][n], sa, sb);
        } else {
          const int64_t g = kt * 4 + j;
          if (g * 128 >= p.K) continue;
          const v4f raw = mfma_raw<FMT>(A.d[mt][j], b);
          const float sbv = sb_rows[(ntile[n] * 16 / 128) * (p.K / 128) + g];
          const float* sa = static_cast<const float*>(p.sa) + g * p.M;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int64_t row = r4[mt] + i < hi ? r4[mt] + i : hi - 1;  // padding rows: any valid scale
            const float f = sa[row] * sbv;
            acc[mt][n][i] = __builtin_fmaf(raw[i], f, acc[mt][n][i]);
          }
        }
      }
    }
  }
}

// Write one 16x16 fp32 tile (lane holds rows 4q+i, col r) to the output or fp32 partials.
__device__ __forceinline__ void store_tile(const GemmParams& p, v4f v, int64_t row0, int64_t row_hi,
                                           int64_t col, int64_t split) {
  if (col >= p.N) return;
  const uint16_t bias = p.bias ? p.bias[col] : (uint16_t)0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = row0 + i;
    if (row >= row_hi) continue;
    if (p.S > 1) {
      p.partial[(split * p.a_rows + row) * p.N + col] = v[i];
    } else {
      p.out[row * p.ldc + col] = out_bits(v[i], p.alpha, p.out_f16, p.bias != nullptr, bias);
    }
  }
}

// Dense: grid (n_groups, m_groups, S), KW waves per workgroup.
// Grouped: grid (n_groups, experts, 1); the workgroup walks its expert's rows.
template <int FMT, int MT, int NT, bool BLOCK, bool GROUPED>
__global__ __launch_bounds__(MT == 1 && NT == 1 ? 1024 : 512) void gemm_kernel(GemmParams p) {
  extern __shared__ float red[];  // [KW][MT][NT][4][64] when KW > 1
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, KW = blockDim.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  // blockIdx.z is the K split, or with two-limb activations (a2 set) the limb:
  // both limbs cover all of K and write fp32 partials that the reduce sums
  const int64_t split = blockIdx.z;
  const bool dual = p.a2 != nullptr;

  const int64_t ntiles_total = (p.N + 15) / 16;
  int64_t ntile[NT], ntile_ld[NT];  // ntile_ld stays inside the packed buffer for a ragged last group
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    ntile[n] = (int64_t)blockIdx.x * NT + n;
    ntile_ld[n] = ntile[n] < ntiles_total ? ntile[n] : ntiles_total - 1;
  }

  int64_t lo = 0, hi = p.M;
  const uint8_t* w = p.w;
  const uint8_t* sw = static_cast<const uint8_t*>(p.sw);
  if (GROUPED) {
    const int64_t e = blockIdx.y;
    lo = p.expert_offsets[e];
    hi = p.expert_offsets[e + 1];
    if (lo >= hi) return;  // experts without routed rows read no weights
    w += e * p.w_expert_stride;
    sw += e * p.sw_expert_stride;
  }
  const int64_t mg_begin = GROUPED ? 0 : (int64_t)blockIdx.y;
  const int64_t mg_end = GROUPED ? (hi - lo + 16 * MT - 1) / (16 * MT) : mg_begin + 1;

  for (int64_t mg = mg_begin; mg < mg_end; ++mg) {
    const int64_t rowbase = lo + mg * 16 * MT;
    int64_t arow[MT], r4[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      int64_t row = rowbase + mt * 16 + (lane >> 2);  // the row this lane loads (row-major loads)
      if (row >= hi) row = hi - 1;  // padding rows reuse a valid row; their outputs are not stored
      arow[mt] = (GROUPED && p.row_index) ? (int64_t)(p.row_index[row] / p.row_div) : row;
      r4[mt] = rowbase + mt * 16 + 4 * q;  // first output row held by this lane
    }
    v4f acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[mt][n] = v4f{0.f, 0.f, 0.f, 0.f};

    // waves take interleaved super-tiles; each super-tile's loads are all issued
    // before its MFMAs wait on them (enough waves per CU keep HBM busy)
    const int64_t kstride = dual ? KW : (int64_t)p.S * KW;
    GemmParams pa = p;
    if (dual && split == 1) {
      pa.a = p.a2;
      pa.sa = p.sa2;
    }
    for (int64_t kt = (dual ? 0 : split * KW) + wv; kt < p.KT; kt += kstride) {
      BTile<FMT, NT> B;
      ATile<MT> A;
      load_b<FMT, NT, BLOCK>(p, w, sw, ntile_ld, kt, lane, B);
      load_a<MT, BLOCK>(pa, arow, kt, lane, A);
      compute_tile<FMT, MT, NT, BLOCK>(p, A, B, acc, kt, q, r4, hi, ntile_ld,
                                       BLOCK ? static_cast<const float*>(p.sw) : nullptr);
    }

    if (KW > 1) {
      float* mine = red + (size_t)wv * (MT * NT * 4 * 64);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
          for (int i = 0; i < 4; ++i) mine[((mt * NT + n) * 4 + i) * 64 + lane] = acc[mt][n][i];
      __syncthreads();
      const int elems = MT * NT * 4 * 64;
      for (int e = threadIdx.x; e < elems; e += blockDim.x) {
        float s = red[e];
        for (int v = 1; v < KW; ++v) s += red[(size_t)v * elems + e];
        const int l = e & 63, i = (e >> 6) & 3, tn = (e >> 8);
        const int n = tn % NT, mt = tn / NT;
        const int64_t row = rowbase + mt * 16 + 4 * (l >> 4) + i;
        const int64_t col = ntile[n] * 16 + (l & 15);
        if (col < p.N && row < hi && ntile[n] < ntiles_total) {
          if (p.S > 1) {
            p.partial[(split * p.a_rows + row) * p.N + col] = s;
          } else {
            p.out[row * p.ldc + col] = out_bits(p, s, col);
          }
        }
      }
      __syncthreads();
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int n = 0; n < NT; ++n)
          if (ntile[n] < ntiles_total)
            store_tile(p, acc[mt][n], rowbase + mt * 16 + 4 * q, hi, ntile[n] * 16 + r, split);
    }
  }
}

// Sum split-K partials in split order, then the output rounding (out_bits: alpha, the
// output format, the bias added after the rounding).
__global__ void splitk_reduce_kernel(const float* __restrict__ partial, const uint16_t* __restrict__ bias,
                                     uint16_t* __restrict__ out, int64_t M, int64_t N, int64_t ldc, int S,
                                     float alpha, int f16) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= M * N) return;
  const int64_t m = id / N, n = id - m * N;
  float s = partial[id];
  for (int k = 1; k < S; ++k) s += partial[(int64_t)k * M * N + id];
  out[m * ldc + n] = out_bits(s, alpha, f16, bias != nullptr, bias ? bias[n] : (uint16_t)0);
}

// The same sum, eight columns per thread (N, ldc multiples of 8, 16-byte aligned
// buffers): two 16-byte loads per split and one 16-byte store, so the pass runs at
// HBM speed instead of being bound by 4-byte accesses.
__global__ __launch_bounds__(256) void splitk_reduce8_kernel(const float* __restrict__ partial,
                                                             const uint16_t* __restrict__ bias,
                                                             uint16_t* __restrict__ out, int64_t M, int64_t N,
                                                             int64_t ldc, int S, float alpha, int f16) {
  const int64_t n8 = N / 8;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= M * n8) return;
  const int64_t m = id / n8, n = (id - m * n8) * 8;
  float4 lo, hi;
  sum_splits8(partial + m * N + n, M * N, S, lo, hi);
  const float f[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  uint32_t h[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const bool b = bias != nullptr;
    const uint16_t h0 = out_bits(f[2 * k], alpha, f16, b, b ? bias[n + 2 * k] : (uint16_t)0);
    const uint16_t h1 = out_bits(f[2 * k + 1], alpha, f16, b, b ? bias[n + 2 * k + 1] : (uint16_t)0);
    h[k] = (uint32_t)h0 | ((uint32_t)h1 << 16);
  }
  *reinterpret_cast<uint4*>(out + m * ldc + n) = uint4{h[0], h[1], h[2], h[3]};
}

// Launch the split-K sum: vectorized when the shapes and buffers allow it.
hipError_t launch_splitk_reduce(const float* partial, const uint16_t* bias, uint16_t* out, int64_t M, int64_t N,
                                int64_t ldc, int S, hipStream_t s, float alpha, int f16) {
  const bool vec = N % 8 == 0 && ldc % 8 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(partial) & 15) == 0;
  if (vec) {
    const int64_t items = M * (N / 8);
    splitk_reduce8_kernel<<<dim3((unsigned)((items + 255) / 256)), 256, 0, s>>>(partial, bias, out, M, N, ldc, S,
                                                                               alpha, f16);
  } else {
    splitk_reduce_kernel<<<dim3((unsigned)((M * N + 255) / 256)), 256, 0, s>>>(partial, bias, out, M, N, ldc, S,
                                                                              alpha, f16);
  }
  return hipGetLastError();
}

// ------------------------------------------------------------ configuration

struct GemmConfig {
  int MT, NT, KW, S;
};

// Choose the wave tile and the K split for an (M, N, K) problem.  Waves of a
// workgroup split K (summed in LDS); workgroups split K further only when the
// output-tile grid alone cannot cover the 256 CUs, since that split costs a
// second launch and an fp32 round trip.
static GemmConfig choose_config(int64_t M, int64_t N, int64_t K) {
  GemmConfig c;
  const int64_t KT = (K + kTileK - 1) / kTileK;
  c.MT = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  c.NT = 1;
  if (M > 32 && M <= 64) { c.MT = 2; c.NT = 2; }
  const int64_t n_groups = ((N + 15) / 16 + c.NT - 1) / c.NT;
  const int64_t m_groups = (M + 16 * c.MT - 1) / (16 * c.MT);
  const int64_t tiles = n_groups * m_groups;
  const int64_t max_kw = (c.MT == 1 && c.NT == 1) ? 16 : 8;
  c.KW = (int)(KT < max_kw ? KT : max_kw);
  int64_t S = 1;
  if (tiles < 128) {
    S = (256 + tiles - 1) / tiles;
    const int64_t max_s = (KT + c.KW - 1) / c.KW;
    if (S > max_s) S = max_s;
  }
  c.S = (int)S;
  return c;
}

template <int FMT, bool BLOCK, bool GROUPED>
static hipError_t launch_gemm(const GemmConfig& c, dim3 grid, const GemmParams& p, hipStream_t stream) {
  const size_t shmem = c.KW > 1 ? (size_t)c.KW * c.MT * c.NT * 4 * 64 * sizeof(float) : 0;
  dim3 block(64 * c.KW);
#define MXL_LAUNCH(MT_, NT_)                                                                        \
  if (c.MT == MT_ && c.NT == NT_) {                                                                 \
    hipLaunchKernelGGL((gemm_kernel<FMT, MT_, NT_, BLOCK, GROUPED>), grid, block, shmem, stream, p); \
    return hipGetLastError();                                                                       \
  }
  MXL_LAUNCH(1, 1)
  // grouped launches use 16-row tiles only (mxl_grouped_gemm's generic schedule)
  if constexpr (!GROUPED) {
    MXL_LAUNCH(2, 1)
    MXL_LAUNCH(4, 1)
    MXL_LAUNCH(2, 2)
  }
#undef MXL_LAUNCH
  return hipErrorInvalidValue;
}

template <bool BLOCK, bool GROUPED>
static hipError_t dispatch_fmt(int fmt, const GemmConfig& c, dim3 grid, const GemmParams& p, hipStream_t s) {
  if (fmt == kE4M3) return launch_gemm<kE4M3, BLOCK, GROUPED>(c, grid, p, s);
  if (BLOCK) return hipErrorInvalidValue;
  if (fmt == kE2M3) return launch_gemm<kE2M3, false, GROUPED>(c, grid, p, s);
  if (fmt == kE3M2) return launch_gemm<kE3M2, false, GROUPED>(c, grid, p, s);
  return hipErrorInvalidValue;
}

}  // namespace mxl

// ------------------------------------------------------------------- C ABI

using namespace mxl;

static bool valid_wfmt(int f) { return f == kE4M3 || f == kE2M3 || f == kE3M2; }

extern "C" int64_t mxl_tiled_weight_bytes(int64_t N, int64_t K, int fmt) {
  const int64_t NTl = (N + 15) / 16, KT = (K + kTileK - 1) / kTileK;
  return NTl * KT * tile_chunks(fmt) * 1024;
}

extern "C" int64_t mxl_tiled_scale_bytes(int64_t N, int64_t K) {
  const int64_t NTl = (N + 15) / 16, KT = (K + kTileK - 1) / kTileK;
  return NTl * KT * 256;
}

static int pack_common(const void* codes, const void* scales, int scale_layout, int64_t N, int64_t K, int fmt,
                       void* tiled_codes, void* tiled_scales, void* stream);

extern "C" int mxl_pack_weight(const void* codes, const void* scales, int64_t N, int64_t K, int fmt,
                               void* tiled_codes, void* tiled_scales, void* stream) {
  return pack_common(codes, scales, 0, N, K, fmt, tiled_codes, tiled_scales, stream);
}

extern "C" int mxl_pack_weight_ex(const void* codes, const void* scales, int scale_layout, int64_t N, int64_t K,
                                  int fmt, void* tiled_codes, void* tiled_scales, void* stream) {
  MXL_CHECK_ARG(scale_layout == 0 || scale_layout == 1, "mxl_pack_weight_ex: unknown scale layout %d", scale_layout);
  return pack_common(codes, scales, scale_layout, N, K, fmt, tiled_codes, tiled_scales, stream);
}

static int pack_common(const void* codes, const void* scales, int scale_layout, int64_t N, int64_t K, int fmt,
                       void* tiled_codes, void* tiled_scales, void* stream) {
  MXL_CHECK_ARG(valid_wfmt(fmt), "mxl_pack_weight: unknown weight format %d", fmt);
  MXL_CHECK_ARG(N > 0 && K > 0 && K % 128 == 0, "mxl_pack_weight: need N > 0 and K %% 128 == 0 (N=%lld K=%lld)",
                (long long)N, (long long)K);
  MXL_CHECK_ARG(((uintptr_t)codes & 15) == 0 && ((uintptr_t)tiled_codes & 15) == 0,
                "mxl_pack_weight: codes must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  const int64_t NTl = (N + 15) / 16, KT = (K + kTileK - 1) / kTileK;
  const int CH = tile_chunks(fmt);
  const int64_t total = NTl * KT * CH * 64;
  const int64_t ld = fmt == kE4M3 ? K : K * 3 / 4;
  pack_weight_kernel<<<dim3((unsigned)((total + 255) / 256)), 256, 0, s>>>(
      (const uint8_t*)codes, ld, (uint8_t*)tiled_codes, N, K, KT, CH, fmt != kE4M3, total);
  MXL_CHECK_LAUNCH("mxl_pack_weight(codes)");
  if (scales) {
    const int64_t ts = NTl * KT * 64;
    pack_scale_kernel<<<dim3((unsigned)((ts + 255) / 256)), 256, 0, s>>>(
        (const uint8_t*)scales, (uint8_t*)tiled_scales, N, K, KT, ts, scale_layout);
    MXL_CHECK_LAUNCH("mxl_pack_weight(scales)");
  }
  return MXL_OK;
}

// The option fields a call may set: anything else is an argument error, not a default.
// An output scale must be finite and non-zero: a zero-filled options struct (alpha 0) is
// a caller's mistake, not a request for zeros.
static bool epilogue_valid(const GemmOptions& o) {
  return (o.out_dtype == kOutBf16 || o.out_dtype == kOutF16) && o.alpha == o.alpha && o.alpha != 0.0f &&
         o.alpha - o.alpha == 0.0f;
}

static bool options_valid(const GemmOptions& o, const char* who) {
  const bool ok = (o.sa_layout == 0 || o.sa_layout == 1) && o.kernel >= kAuto && o.kernel <= kChunk &&
                  o.splits >= 0 && o.splits <= 64 && (o.tile_n == 0 || o.tile_n == 1 || o.tile_n == 2 ||
                  o.tile_n == 4) && (o.tile_m == 0 || o.tile_m == 4 || o.tile_m == 8) &&
                  (o.hybrid == 0 || o.hybrid == 1) && (o.waves == 0 || o.waves == 4 || o.waves == 8) &&
                  epilogue_valid(o);
  if (!ok)
    set_error("%s: invalid options {sa_layout %d, kernel %d, splits %d, tile_n %d, tile_m %d, hybrid %d, waves %d, "
              "out_dtype %d, alpha %g} (alpha must be finite and non-zero: 1 for no scaling)",
              who, o.sa_layout, o.kernel, o.splits, o.tile_n, o.tile_m, o.hybrid, o.waves, o.out_dtype,
              (double)o.alpha);
  return ok;
}

// The C ABI's mxl_gemm_options (include/mxlinear.h), field for field.
struct AbiGemmOptions {
  int sa_layout, kernel, splits, tile_n, tile_m, hybrid, waves, out_dtype;
  float alpha;
};

static GemmOptions options_of(const void* opts) {
  GemmOptions o;
  if (opts) {
    const AbiGemmOptions& v = *static_cast<const AbiGemmOptions*>(opts);
    o.sa_layout = v.sa_layout; o.kernel = v.kernel; o.splits = v.splits; o.tile_n = v.tile_n; o.tile_m = v.tile_m;
    o.hybrid = v.hybrid; o.waves = v.waves; o.out_dtype = v.out_dtype; o.alpha = v.alpha;
  }
  return o;
}

static bool default_epilogue(const GemmOptions& o) { return o.out_dtype == kOutBf16 && o.alpha == 1.0f; }

// The dense kernel and split a call runs with (shared by the launch and the workspace
// query, so that the bytes the query reports are the bytes the launch uses).
struct DensePlan {
  int kernel;  // kStream, kWide, kGeneric or kChunk
  WideConfig wide{2, 1, 1};
  GemmConfig gen{};
  int64_t need = 0;  // split-K workspace bytes of the plan
};

// ------------------------------------------------------------ per-shape plan overrides
//
// A measured per-shape table replaces the cost model's choice for exact (M, N, K, weight
// format, block) shapes on one device: the role of the reference's registered projection
// configs (src/vllm_mach/mxfp6/moe_projection.py:35-105, set_w6a8_config per table row).
// An entry holds the tuning fields (kernel, splits, tile_n, tile_m, hybrid, waves); a call
// whose own tuning fields are all automatic takes them, its scale layout and epilogue
// unchanged.  Lookups cost one relaxed atomic load while the table is empty.
namespace {
constexpr int64_t kGemmConfigAbi = 1;  // the fields and kernel ids an entry may name
constexpr int64_t kGemmConfigMax = 4096;

struct ShapeKey {
  int dev;
  int64_t M, N, K;
  int fmt, block;
  bool operator==(const ShapeKey& b) const {
    return dev == b.dev && M == b.M && N == b.N && K == b.K && fmt == b.fmt && block == b.block;
  }
};
struct ShapeKeyHash {
  size_t operator()(const ShapeKey& k) const {
    uint64_t h = 1469598103934665603ull;
    const int64_t v[6] = {k.dev, k.M, k.N, k.K, k.fmt, k.block};
    for (int64_t x : v) h = (h ^ (uint64_t)x) * 1099511628211ull;
    return (size_t)h;
  }
};
std::mutex g_cfg_mu;
std::unordered_map<ShapeKey, GemmOptions, ShapeKeyHash> g_cfg;
std::atomic<int64_t> g_cfg_count{0};

int config_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;  // no device (host-side planning): device 0
  return dev;
}

bool tuning_auto(const GemmOptions& o) {
  return o.kernel == kAuto && o.splits == 0 && o.tile_n == 0 && o.tile_m == 0 && o.hybrid == 0 && o.waves == 0;
}

// o with the registered tuning fields of this shape, when o leaves them automatic
GemmOptions with_override(int64_t M, int64_t N, int64_t K, int fmt, bool block, const GemmOptions& o) {
  if (g_cfg_count.load(std::memory_order_relaxed) == 0 || !tuning_auto(o)) return o;
  const ShapeKey key{config_device(), M, N, K, fmt, block ? 1 : 0};
  std::lock_guard<std::mutex> lock(g_cfg_mu);
  const auto it = g_cfg.find(key);
  if (it == g_cfg.end()) return o;
  GemmOptions r = o;
  r.kernel = it->second.kernel;
  r.splits = it->second.splits;
  r.tile_n = it->second.tile_n;
  r.tile_m = it->second.tile_m;
  r.hybrid = it->second.hybrid;
  r.waves = it->second.waves;
  return r;
}
}  // namespace

static bool plan_dense_as(int64_t M, int64_t N, int64_t K, int fmt, bool block, const GemmOptions& o,
                          DensePlan& d);

static bool plan_dense(int64_t M, int64_t N, int64_t K, int fmt, bool block, const GemmOptions& o, DensePlan& d) {
  return plan_dense_as(M, N, K, fmt, block, with_override(M, N, K, fmt, block, o), d);
}

static bool plan_dense_as(int64_t M, int64_t N, int64_t K, int fmt, bool block, const GemmOptions& o,
                          DensePlan& d) {
  const bool stream_ok = stream_gemm_eligible(M, K, block);
  const bool wide_ok = wide_gemm_eligible(M, K) && (!block || K <= int64_t(128) * kWideBlockStages);
  const bool chunk_ok = !block && chunk_gemm_eligible(M, K, fmt);
  // Short K over few n-tiles: the generic kernel splits K over the waves of one workgroup
  // and writes bf16 directly, where the wide kernel needs a K split and its reduce to fill
  // the CUs.  Measured by a per-shape sweep over every kernel, tile and split (µs, generic
  // against the wide or K-chunked pick): MXFP8 2048 x 2048 at M = 64 / 128 / 256 6.5 /
  // 7.5 / 8.5 against 8.6 / 8.7 / 13.0, W6A8 N = 512 and 2048, K = 2048 at M = 64..128
  // 5.9-7.2 against 8.1-8.4.
  const bool generic_pref = !block && M > 32 && M <= 256 && K >= 1024 && K <= 2048 && (N + 15) / 16 <= 128;
  d.kernel = o.kernel == kAuto
                 ? (stream_ok                                        ? kStream
                    : chunk_ok && chunk_gemm_preferred(M, N, K)      ? kChunk
                    : generic_pref || !wide_ok                       ? kGeneric
                                                                     : kWide)
                 : o.kernel;
  if ((d.kernel == kStream && !stream_ok) || (d.kernel == kWide && !wide_ok) || (d.kernel == kChunk && !chunk_ok) ||
      (d.kernel != kStream && d.kernel != kWide && d.kernel != kGeneric && d.kernel != kChunk))
    return false;
  if (d.kernel == kChunk) {
    const int64_t nch = chunk_count(K, kChunkSuperTiles);
    d.need = nch > 1 ? nch * M * N * 4 : 0;
    return true;
  }
  if (d.kernel == kWide) {
    if (block && o.tile_n == 0 && o.waves == 0 && o.splits == 0 && !o.hybrid && o.tile_m == 0) {
      // Block-FP8: eight waves (two per SIMD, so one wave's per-K128 folds run under the
      // other's MFMAs) on 128 x 128 tiles, which fit their registers.  Measured at c3 (N =
      // 18432, K = 2560; µs, four-wave pick -> this): M = 128 23.4 -> 20.3, M = 256 37.2 ->
      // 33.7 (one full round plus split remainder), M = 512 58.6 -> 55.5 (three rounds: the
      // split remainder after two full rounds measured 63.7).
      // At most 64 rows: 64-row tiles on four waves (c3 M = 64: 16.2 against 19.7 µs for
      // half-empty 128-row tiles on eight).
      GemmOptions o2 = o;
      o2.tile_n = 2;
      if (M <= 64) o2.tile_m = 4;
      d.wide = wide_config(M, N, K, fmt, o2);
      if (d.wide.dp_tiles >= 2 * (int64_t)cu_count()) {
        const int mt = d.wide.MT;
        d.wide = WideConfig{2, 1, (K + kTileK - 1) / kTileK};
        d.wide.MT = mt;
      }
      d.wide.WM = d.wide.MT == 8 ? 2 : 1;
    } else {
      d.wide = wide_config(M, N, K, fmt, o);
      if (block && d.wide.NT == 4) d.wide.WM = 1;  // no eight-wave block-FP8 tile of four n-tiles per wave
      // MX 128 x 128 tiles: eight waves, bit-identical, measured 1-3 % faster where the
      // model picks them (c2 M = 512 29.2 -> 28.5 µs, c4 M = 128 35.1 -> 34.0, M = 256
      // 46.5 -> 46.2); 64-column tiles measured slower with eight waves
      const bool auto_tile = o.tile_n == 0 && o.splits == 0 && o.waves == 0 && o.tile_m == 0 && !o.hybrid;
      if (!block && auto_tile && d.wide.NT == 2 && d.wide.MT == 8) d.wide.WM = 2;
    }
    d.need = wide_workspace_bytes(d.wide, M, N);
  } else if (d.kernel == kGeneric) {
    d.gen = choose_config(M, N, K);
    if (o.splits >= 1 && o.kernel == kGeneric) d.gen.S = o.splits;
    d.need = d.gen.S > 1 ? (int64_t)d.gen.S * M * N * 4 : 0;
  }
  return true;
}

static int gemm_common(const void* a, const void* sa, int64_t M, const void* w_tiled, const void* sw, int64_t N,
                       int64_t K, int fmt, bool block, const void* bias, void* out, int64_t ldc, void* workspace,
                       int64_t workspace_bytes, const GemmOptions& o, void* stream, const char* who) {
  MXL_CHECK_ARG(M >= 0 && N > 0 && K > 0 && K % 128 == 0, "%s: need N > 0, K %% 128 == 0 (M=%lld N=%lld K=%lld)", who,
                (long long)M, (long long)N, (long long)K);
  MXL_CHECK_ARG(ldc >= N, "%s: ldc < N", who);
  MXL_CHECK_ARG(((uintptr_t)a & 15) == 0 && ((uintptr_t)w_tiled & 15) == 0, "%s: a and w must be 16-byte aligned", who);
  MXL_CHECK_ARG(o.sa_layout == 0 || (o.sa_layout == 1 && !block), "%s: unknown activation scale layout %d", who,
                o.sa_layout);
  MXL_CHECK_ARG(o.splits >= 0 && o.splits <= 64, "%s: splits must be 0 (automatic) .. 64", who);
  if (!options_valid(o, who)) return MXL_EINVAL;
  if (M == 0) return MXL_OK;
  DensePlan d;
  if (!plan_dense(M, N, K, fmt, block, o, d)) {
    set_error("%s: kernel %d does not run (M=%lld, K=%lld)", who, o.kernel, (long long)M, (long long)K);
    return MXL_EUNSUPPORTED;
  }
  GemmParams p{};
  p.a = (const uint8_t*)a; p.sa = sa; p.w = (const uint8_t*)w_tiled; p.sw = sw;
  p.bias = (const uint16_t*)bias; p.out = (uint16_t*)out; p.partial = (float*)workspace;
  p.lda = K; p.ldc = ldc; p.M = M; p.N = N; p.K = K; p.KT = (K + kTileK - 1) / kTileK; p.a_rows = M;
  p.row_div = 1;
  p.alpha = o.alpha;
  p.out_f16 = o.out_dtype == kOutF16;
  set_sa_layout(p, o.sa_layout);
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  const bool room = d.need == 0 || (workspace != nullptr && d.need <= workspace_bytes);
  if (d.kernel == kStream) {
    p.S = 1;
    e = launch_gemm_stream(fmt, block, p, s);
  } else if (d.kernel == kChunk) {
    if (!room) {
      set_error("%s: the K-chunked kernel needs %lld bytes of workspace (have %lld)", who, (long long)d.need,
                (long long)workspace_bytes);
      return MXL_EINVAL;
    }
    p.S = (int)chunk_count(K, kChunkSuperTiles);
    e = launch_gemm_chunk(fmt, p, s);
  } else if (d.kernel == kWide) {
    WideConfig wc = d.wide;
    if (!room) {
      const int mt = wc.MT;
      wc = WideConfig{wc.NT, 1, (K + kTileK - 1) / kTileK};  // no room: skip the K split
      wc.MT = mt;
    }
    p.S = wc.S;
    e = launch_gemm_wide(fmt, block, wc, p, 0, s);
  } else {
    GemmConfig c = d.gen;
    if (!room) c.S = 1;
    p.S = c.S;
    const int64_t n_groups = ((N + 15) / 16 + c.NT - 1) / c.NT;
    const int64_t m_groups = (M + 16 * c.MT - 1) / (16 * c.MT);
    dim3 grid((unsigned)n_groups, (unsigned)m_groups, (unsigned)c.S);
    e = block ? dispatch_fmt<true, false>(fmt, c, grid, p, s) : dispatch_fmt<false, false>(fmt, c, grid, p, s);
  }
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", who, hipGetErrorString(e));
    return MXL_EHIP;
  }
  if (p.S > 1 && d.kernel != kWide) {  // (the wide kernel's launch runs its own tile reduce)
    e = launch_splitk_reduce((const float*)workspace, (const uint16_t*)bias, (uint16_t*)out, M, N, ldc, p.S, s,
                             p.alpha, p.out_f16);
    if (e != hipSuccess) {
      set_error("%s: split-K reduce launch failed: %s", who, hipGetErrorString(e));
      return MXL_EHIP;
    }
  }
  return MXL_OK;
}

extern "C" int64_t mxl_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 128) return 0;
  // the largest need over the weight formats and the block-FP8 mode
  int64_t bytes = 0;
  for (int fmt : {kE4M3, kE2M3}) {
    DensePlan d;
    if (plan_dense(M, N, K, fmt, false, GemmOptions(), d) && d.need > bytes) bytes = d.need;
  }
  DensePlan d;
  if (plan_dense(M, N, K, kE4M3, true, GemmOptions(), d) && d.need > bytes) bytes = d.need;
  return bytes;
}

extern "C" int64_t mxl_gemm_workspace_bytes_ex(int64_t M, int64_t N, int64_t K, int w_fmt, int block,
                                               const void* options) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 128 || !valid_wfmt(w_fmt)) return 0;
  DensePlan d;
  return plan_dense(M, N, K, w_fmt, block != 0, options_of(options), d) ? d.need : 0;
}

extern "C" int64_t mxl_gemm_config_abi(void) { return kGemmConfigAbi; }

extern "C" int64_t mxl_gemm_config_count(void) { return g_cfg_count.load(std::memory_order_relaxed); }

extern "C" int mxl_set_gemm_config(int64_t M, int64_t N, int64_t K, int w_fmt, int block, const void* options) {
  const char* who = "mxl_set_gemm_config";
  MXL_CHECK_ARG(valid_wfmt(w_fmt), "%s: unknown weight format %d", who, w_fmt);
  MXL_CHECK_ARG(M > 0 && N > 0 && K > 0 && K % 128 == 0, "%s: need M, N, K > 0 and K %% 128 == 0 (M=%lld N=%lld K=%lld)",
                who, (long long)M, (long long)N, (long long)K);
  MXL_CHECK_ARG(options != nullptr, "%s: options must not be NULL", who);
  const GemmOptions o = options_of(options);
  if (!options_valid(o, who)) return MXL_EINVAL;
  DensePlan d;
  MXL_CHECK_ARG(plan_dense_as(M, N, K, w_fmt, block != 0, o, d),
                "%s: the options {kernel %d, splits %d, tile_n %d, tile_m %d, hybrid %d, waves %d} do not run "
                "M=%lld N=%lld K=%lld (format %d, block %d)",
                who, o.kernel, o.splits, o.tile_n, o.tile_m, o.hybrid, o.waves, (long long)M, (long long)N,
                (long long)K, w_fmt, block);
  const ShapeKey key{config_device(), M, N, K, w_fmt, block ? 1 : 0};
  std::lock_guard<std::mutex> lock(g_cfg_mu);
  if (g_cfg.find(key) == g_cfg.end() && (int64_t)g_cfg.size() >= kGemmConfigMax) {
    set_error("%s: the table holds at most %lld shapes", who, (long long)kGemmConfigMax);
    return MXL_EINVAL;
  }
  g_cfg[key] = o;
  g_cfg_count.store((int64_t)g_cfg.size(), std::memory_order_relaxed);
  return MXL_OK;
}

extern "C" int mxl_clear_gemm_configs(void) {
  std::lock_guard<std::mutex> lock(g_cfg_mu);
  g_cfg.clear();
  g_cfg_count.store(0, std::memory_order_relaxed);
  return MXL_OK;
}

extern "C" int mxl_mx_gemm(const void* a, const void* sa, int64_t M, const void* w_tiled, const void* sw_tiled,
                           int64_t N, int64_t K, int w_fmt, const void* bias, void* out, int64_t ldc,
                           void* workspace, int64_t workspace_bytes, void* stream) {
  MXL_CHECK_ARG(valid_wfmt(w_fmt), "mxl_mx_gemm: unknown weight format %d", w_fmt);
  return gemm_common(a, sa, M, w_tiled, sw_tiled, N, K, w_fmt, false, bias, out, ldc, workspace, workspace_bytes,
                     GemmOptions(), stream, "mxl_mx_gemm");
}

extern "C" int mxl_mx_gemm_ex(const void* a, const void* sa, int64_t M, const void* w_tiled, const void* sw_tiled,
                              int64_t N, int64_t K, int w_fmt, const void* bias, void* out, int64_t ldc,
                              void* workspace, int64_t workspace_bytes, const void* options, void* stream) {
  MXL_CHECK_ARG(valid_wfmt(w_fmt), "mxl_mx_gemm_ex: unknown weight format %d", w_fmt);
  return gemm_common(a, sa, M, w_tiled, sw_tiled, N, K, w_fmt, false, bias, out, ldc, workspace, workspace_bytes,
                     options_of(options), stream, "mxl_mx_gemm_ex");
}

// ------------------------------------------------------ no-allocation entry point

// Split-K scratch of mxl_mx_gemm_noalloc.  Every GPU that loads this code object
// holds its own copy until the process ends.  On the host `scratch` names a
// stand-in, not a device address: host code uses only the per-device address that
// hipGetSymbolAddress returns (g_scratch_ptr), never the array's name.
constexpr int64_t kNoAllocScratchBytes = int64_t(32) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, queried once per device (with that
// device current) and kept.
int scratch_address(const char* who, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("%s: no current HIP device (%s)", who, hipGetErrorString(e));
    return MXL_EHIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev, hipGetErrorString(e));
      return MXL_EHIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MXL_OK;
}
}  // namespace

extern "C" int64_t mxl_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int mxl_mx_gemm_noalloc(const void* a, const void* sa, int64_t M, const void* w_tiled,
                                   const void* sw_tiled, int64_t N, int64_t K, int w_fmt, const void* bias, void* out,
                                   int64_t ldc, void* stream) {
  const char* who = "mxl_mx_gemm_noalloc";
  MXL_CHECK_ARG(valid_wfmt(w_fmt), "%s: unknown weight format %d", who, w_fmt);
  MXL_CHECK_ARG(M >= 0 && N > 0 && K > 0 && K % 128 == 0, "%s: need N > 0, K %% 128 == 0 (M=%lld N=%lld K=%lld)", who,
                (long long)M, (long long)N, (long long)K);
  if (M == 0) return MXL_OK;
  // the plan mxl_mx_gemm makes for this shape; its split-K partials must fit the scratch
  DensePlan d;
  if (!plan_dense(M, N, K, w_fmt, false, GemmOptions(), d)) {
    set_error("%s: no kernel runs this shape (M=%lld, K=%lld)", who, (long long)M, (long long)K);
    return MXL_EUNSUPPORTED;
  }
  MXL_CHECK_ARG(d.need <= kNoAllocScratchBytes,
                "%s: this shape needs %lld bytes of split-K scratch, more than the %lld this entry point holds "
                "(M=%lld N=%lld K=%lld); use mxl_mx_gemm with a workspace",
                who, (long long)d.need, (long long)kNoAllocScratchBytes, (long long)M, (long long)N, (long long)K);
  if (stream) {  // the scratch is the current device's: the stream must belong to it
    int cur = -1, sdev = -1;
    if (hipGetDevice(&cur) != hipSuccess || hipStreamGetDevice((hipStream_t)stream, &sdev) != hipSuccess ||
        cur != sdev) {
      set_error("%s: the stream's device (%d) is not the current device (%d)", who, sdev, cur);
      return MXL_EINVAL;
    }
  }
  void* ws = nullptr;
  const int rc = scratch_address(who, &ws);
  if (rc != MXL_OK) return rc;
  return gemm_common(a, sa, M, w_tiled, sw_tiled, N, K, w_fmt, false, bias, out, ldc, ws, kNoAllocScratchBytes,
                     GemmOptions(), stream, who);
}

static int swiglu_row_common(const void* gate_up, int64_t M, int64_t K, int rule, const void* w_tiled,
                             const void* sw_tiled, int64_t N, int w_fmt, const void* bias, void* out, int64_t ldc,
                             const GemmOptions& o, void* stream) {
  MXL_CHECK_ARG(valid_wfmt(w_fmt), "mxl_swiglu_mx_gemm: unknown weight format %d", w_fmt);
  MXL_CHECK_ARG(epilogue_valid(o), "mxl_swiglu_mx_gemm: output format %d / alpha %g invalid", o.out_dtype,
                (double)o.alpha);
  MXL_CHECK_ARG(N > 0 && ldc >= N, "mxl_swiglu_mx_gemm: need N > 0 and ldc >= N");
  MXL_CHECK_ARG(((uintptr_t)gate_up & 15) == 0 && ((uintptr_t)w_tiled & 15) == 0,
                "mxl_swiglu_mx_gemm: gate_up and w must be 16-byte aligned");
  const bool rule_ok = rule == kCeilDiv448 || rule == kRpUe8m0;
  const bool handoff = rule_ok && stream_fused_eligible(M, K, false, w_fmt);
  const bool rowwise = stream_swiglu_eligible(M, K, rule);
  // automatic: the row recomputed by every wavefront where it runs (M = 1: measured faster
  // than the handoff, whose grid-wide synchronisation costs more than the launch it saves)
  const bool use_rowwise = o.kernel == kStreamWide || (o.kernel == kAuto && rowwise);
  if (use_rowwise ? !rowwise : (!handoff || (o.kernel != kAuto && o.kernel != kStream))) {
    set_error("mxl_swiglu_mx_gemm: unsupported (M <= 16, K %% 128 == 0, K <= 12288 except 7680 < K <= 8192 and "
              "K > 11264 for M > 1, rule 1 or 2; options.kernel -1, 0 or 3 (3: M = 1); M=%lld K=%lld rule=%d "
              "kernel=%d)", (long long)M, (long long)K, rule, o.kernel);
    return MXL_EUNSUPPORTED;
  }
  if (M == 0) return MXL_OK;
  GemmParams p{};
  p.a = (const uint8_t*)gate_up;
  p.w = (const uint8_t*)w_tiled; p.sw = sw_tiled; p.bias = (const uint16_t*)bias; p.out = (uint16_t*)out;
  p.lda = 2 * K; p.ldc = ldc; p.M = M; p.N = N; p.K = K; p.KT = (K + kTileK - 1) / kTileK; p.a_rows = M;
  p.row_div = 1; p.S = 1;
  p.alpha = o.alpha; p.out_f16 = o.out_dtype == kOutF16;
  if (!use_rowwise) {
    p.fsrc = (const uint16_t*)gate_up;
    p.fsrc_ld = 2 * K;
    return launch_gemm_stream_fused(w_fmt, rule, p, (hipStream_t)stream, "mxl_swiglu_mx_gemm");
  }
  const hipError_t e = launch_gemm_stream_swiglu(w_fmt, rule, p, (hipStream_t)stream);
  if (e != hipSuccess) {
    set_error("mxl_swiglu_mx_gemm: launch failed: %s", hipGetErrorString(e));
    return MXL_EHIP;
  }
  return MXL_OK;
}

extern "C" int mxl_swiglu_mx_gemm(const void* gate_up, int64_t M, int64_t K, int rule, const void* w_tiled,
                                  const void* sw_tiled, int64_t N, int w_fmt, const void* bias, void* out,
                                  int64_t ldc, void* stream) {
  return swiglu_row_common(gate_up, M, K, rule, w_tiled, sw_tiled, N, w_fmt, bias, out, ldc, GemmOptions(), stream);
}

extern "C" int mxl_swiglu_mx_gemm_ex(const void* gate_up, int64_t M, int64_t K, int rule, const void* w_tiled,
                                     const void* sw_tiled, int64_t N, int w_fmt, const void* bias, void* out,
                                     int64_t ldc, const void* options, void* stream) {
  return swiglu_row_common(gate_up, M, K, rule, w_tiled, sw_tiled, N, w_fmt, bias, out, ldc, options_of(options),
                           stream);
}

static int quant_row_common(const void* x, int64_t M, int64_t K, int rule, const void* w_tiled, const void* sw_tiled,
                            int64_t N, int w_fmt, const void* bias, void* out, int64_t ldc, const GemmOptions& o,
                            void* stream) {
  MXL_CHECK_ARG(valid_wfmt(w_fmt), "mxl_quant_mx_gemm: unknown weight format %d", w_fmt);
  MXL_CHECK_ARG(epilogue_valid(o), "mxl_quant_mx_gemm: output format %d / alpha %g invalid", o.out_dtype,
                (double)o.alpha);
  MXL_CHECK_ARG(N > 0 && ldc >= N, "mxl_quant_mx_gemm: need N > 0 and ldc >= N");
  MXL_CHECK_ARG(((uintptr_t)x & 15) == 0 && ((uintptr_t)w_tiled & 15) == 0,
                "mxl_quant_mx_gemm: x and w must be 16-byte aligned");
  const bool rule_ok = rule >= kFloorCarry175 && rule <= kRpUe8m0;
  const bool handoff = rule_ok && stream_fused_eligible(M, K, false, w_fmt);
  const bool rowwise = stream_quant_row_eligible(M, K, rule);
  const bool qrows = stream_quant_rows_eligible(M, K, rule);
  // The producer inside the GEMM's own wavefronts (options.kernel 3, automatic where it
  // runs): for one row every wavefront quantizes its super-tiles' row values; for up to 16
  // rows (K <= 6144) every fragment lane its own pieces, once per workgroup.  Both measured
  // faster than the producer waves' grid-wide handoff (options.kernel 0), whose
  // synchronisation costs more than the launch it saves.
  const bool inreg = M == 1 ? rowwise : qrows;
  const bool use_inreg = o.kernel == kStreamWide || (o.kernel == kAuto && inreg);
  if (use_inreg ? !inreg : (!handoff || (o.kernel != kAuto && o.kernel != kStream))) {
    set_error("mxl_quant_mx_gemm: unsupported (M <= 16, K %% 128 == 0, K <= 12288 except 7680 < K <= 8192 and "
              "K > 11264 for M > 1, rule 0, 1 or 2; options.kernel -1, 0 or 3 (3: M = 1, or M <= 16 with "
              "K <= 6144); M=%lld K=%lld rule=%d kernel=%d)", (long long)M, (long long)K, rule, o.kernel);
    return MXL_EUNSUPPORTED;
  }
  if (M == 0) return MXL_OK;
  GemmParams p{};
  p.a = (const uint8_t*)x;
  p.w = (const uint8_t*)w_tiled; p.sw = sw_tiled; p.bias = (const uint16_t*)bias; p.out = (uint16_t*)out;
  p.lda = K; p.ldc = ldc; p.M = M; p.N = N; p.K = K; p.KT = (K + kTileK - 1) / kTileK; p.a_rows = M;
  p.row_div = 1; p.S = 1;
  p.alpha = o.alpha; p.out_f16 = o.out_dtype == kOutF16;
  if (!use_inreg) {
    p.fsrc = (const uint16_t*)x;
    p.fsrc_ld = K;
    return launch_gemm_stream_fused(w_fmt, 4 + rule, p, (hipStream_t)stream, "mxl_quant_mx_gemm");
  }
  const hipError_t e = M == 1 ? launch_gemm_stream_quant_row(w_fmt, rule, p, (hipStream_t)stream)
                              : launch_gemm_stream_quant_rows(w_fmt, rule, p, (hipStream_t)stream);
  if (e != hipSuccess) {
    set_error("mxl_quant_mx_gemm: launch failed: %s", hipGetErrorString(e));
    return MXL_EHIP;
  }
  return MXL_OK;
}

extern "C" int mxl_quant_mx_gemm(const void* x, int64_t M, int64_t K, int rule, const void* w_tiled,
                                 const void* sw_tiled, int64_t N, int w_fmt, const void* bias, void* out, int64_t ldc,
                                 void* stream) {
  return quant_row_common(x, M, K, rule, w_tiled, sw_tiled, N, w_fmt, bias, out, ldc, GemmOptions(), stream);
}

extern "C" int mxl_quant_mx_gemm_ex(const void* x, int64_t M, int64_t K, int rule, const void* w_tiled,
                                    const void* sw_tiled, int64_t N, int w_fmt, const void* bias, void* out,
                                    int64_t ldc, const void* options, void* stream) {
  return quant_row_common(x, M, K, rule, w_tiled, sw_tiled, N, w_fmt, bias, out, ldc, options_of(options), stream);
}

extern "C" int mxl_producer_gemm_supported(int kind, int64_t M, int64_t K, int rule, int w_fmt) {
  if (M < 0 || K <= 0) return 0;
  const int64_t m = M > 0 ? M : 1;
  switch (kind) {
    case 0:  // SwiGLU -> MXFP8 -> MX GEMM
      return valid_wfmt(w_fmt) && (rule == kCeilDiv448 || rule == kRpUe8m0) &&
             (stream_fused_eligible(m, K, false, w_fmt) || stream_swiglu_eligible(m, K, rule));
    case 1:  // MXFP8 quantization -> MX GEMM
      return valid_wfmt(w_fmt) && rule >= kFloorCarry175 && rule <= kRpUe8m0 &&
             (stream_fused_eligible(m, K, false, w_fmt) || stream_quant_row_eligible(m, K, rule) ||
              stream_quant_rows_eligible(m, K, rule));
    case 2:  // block-FP8 quantization -> block-FP8 GEMM
      return stream_fused_eligible(m, K, true, kE4M3) || stream_block_row_eligible(m, K);
    case 4:  // block-FP8 quantization inside the GEMM's own wavefronts (one row)
      return stream_block_row_eligible(m, K);
    case 3:  // MXFP8 quantization inside the GEMM's own wavefronts (no handoff)
      return valid_wfmt(w_fmt) && (m == 1 ? stream_quant_row_eligible(1, K, rule) : stream_quant_rows_eligible(m, K, rule));
    default:
      return 0;
  }
}

// Block-FP8 activation quantization + block-FP8 GEMM in one launch (M <= 16).
static int block_quant_common(const void* x, int64_t M, int64_t K, const void* w_tiled, const void* sb, int64_t N,
                              const void* bias, void* out, int64_t ldc, const GemmOptions& o, void* stream) {
  MXL_CHECK_ARG(N > 0 && ldc >= N && K > 0 && K % 128 == 0 && M >= 0,
                "mxl_block_fp8_quant_gemm: need M >= 0, N > 0, ldc >= N, K %% 128 == 0");
  MXL_CHECK_ARG(epilogue_valid(o), "mxl_block_fp8_quant_gemm: output format %d / alpha %g invalid", o.out_dtype,
                (double)o.alpha);
  MXL_CHECK_ARG(((uintptr_t)x & 15) == 0 && ((uintptr_t)w_tiled & 15) == 0,
                "mxl_block_fp8_quant_gemm: x and w must be 16-byte aligned");
  // one row: every wavefront quantizes it (options.kernel 3, automatic where it runs);
  // more rows: the producer waves' grid handoff (options.kernel 0)
  const bool inreg = stream_block_row_eligible(M, K);
  const bool handoff = stream_fused_eligible(M > 0 ? M : 1, K, true, kE4M3);
  const bool use_inreg = o.kernel == kStreamWide || (o.kernel == kAuto && inreg);
  if (use_inreg ? !inreg : (!handoff || (o.kernel != kAuto && o.kernel != kStream))) {
    set_error("mxl_block_fp8_quant_gemm: unsupported (M <= 16, K %% 128 == 0, K <= 3584 or 4096 < K <= 7168; "
              "options.kernel -1, 0 or 3 (3: M = 1, K <= 8192); M=%lld K=%lld kernel=%d)", (long long)M, (long long)K,
              o.kernel);
    return MXL_EUNSUPPORTED;
  }
  if (M == 0) return MXL_OK;
  GemmParams p{};
  p.w = (const uint8_t*)w_tiled; p.sw = sb; p.bias = (const uint16_t*)bias; p.out = (uint16_t*)out;
  p.ldc = ldc; p.M = M; p.N = N; p.K = K; p.KT = (K + kTileK - 1) / kTileK; p.a_rows = M;
  p.row_div = 1; p.S = 1;
  p.alpha = o.alpha; p.out_f16 = o.out_dtype == kOutF16;
  if (use_inreg) {
    p.a = (const uint8_t*)x;
    p.lda = K;
    const hipError_t e = launch_gemm_stream_block_row(p, (hipStream_t)stream);
    if (e != hipSuccess) {
      set_error("mxl_block_fp8_quant_gemm: launch failed: %s", hipGetErrorString(e));
      return MXL_EHIP;
    }
    return MXL_OK;
  }
  p.fsrc = (const uint16_t*)x;
  p.fsrc_ld = K;
  return launch_gemm_stream_fused(kE4M3, kFusedBlockFp8, p, (hipStream_t)stream, "mxl_block_fp8_quant_gemm");
}

extern "C" int mxl_block_fp8_quant_gemm(const void* x, int64_t M, int64_t K, const void* w_tiled, const void* sb,
                                        int64_t N, const void* bias, void* out, int64_t ldc, void* stream) {
  return block_quant_common(x, M, K, w_tiled, sb, N, bias, out, ldc, GemmOptions(), stream);
}

extern "C" int mxl_block_fp8_quant_gemm_ex(const void* x, int64_t M, int64_t K, const void* w_tiled, const void* sb,
                                           int64_t N, const void* bias, void* out, int64_t ldc, const void* options,
                                           void* stream) {
  return block_quant_common(x, M, K, w_tiled, sb, N, bias, out, ldc, options_of(options), stream);
}

static int gemm_dual_common(const void* hi, const void* s_hi, const void* res, const void* s_res, int64_t M,
                            const void* w_tiled, const void* sw_tiled, int64_t N, int64_t K, int w_fmt,
                            const void* bias, void* out, int64_t ldc, void* workspace, int64_t workspace_bytes,
                            const GemmOptions& o, void* stream) {
  MXL_CHECK_ARG(valid_wfmt(w_fmt), "mxl_mx_gemm_dual: unknown weight format %d", w_fmt);
  MXL_CHECK_ARG(o.sa_layout == 0 || o.sa_layout == 1, "mxl_mx_gemm_dual: sa_layout must be 0 or 1");
  if (!options_valid(o, "mxl_mx_gemm_dual")) return MXL_EINVAL;
  MXL_CHECK_ARG(default_epilogue(o), "mxl_mx_gemm_dual: bf16 output without scaling only");
  MXL_CHECK_ARG(M >= 0 && M <= 64 && N > 0 && K > 0 && K % 128 == 0,
                "mxl_mx_gemm_dual: need M <= 64, N > 0, K %% 128 == 0 (M=%lld N=%lld K=%lld)", (long long)M,
                (long long)N, (long long)K);
  MXL_CHECK_ARG(ldc >= N, "mxl_mx_gemm_dual: ldc < N");
  MXL_CHECK_ARG(((uintptr_t)hi & 15) == 0 && ((uintptr_t)res & 15) == 0 && ((uintptr_t)w_tiled & 15) == 0,
                "mxl_mx_gemm_dual: hi, res and w must be 16-byte aligned");
  MXL_CHECK_ARG(workspace && workspace_bytes >= 2 * M * N * 4,
                "mxl_mx_gemm_dual: workspace too small (%lld < %lld)", (long long)workspace_bytes,
                (long long)(2 * M * N * 4));
  if (M == 0) return MXL_OK;
  GemmParams p{};
  p.a = (const uint8_t*)hi; p.sa = s_hi; p.a2 = (const uint8_t*)res; p.sa2 = s_res;
  p.w = (const uint8_t*)w_tiled; p.sw = sw_tiled; p.bias = (const uint16_t*)bias; p.out = (uint16_t*)out;
  p.partial = (float*)workspace;
  p.lda = K; p.ldc = ldc; p.M = M; p.N = N; p.K = K; p.KT = (K + kTileK - 1) / kTileK; p.a_rows = M;
  p.row_div = 1;
  set_sa_layout(p, o.sa_layout);
  p.S = 2;  // the two limbs' fp32 partials
  GemmConfig c = choose_config(M, N, K);
  c.S = 1;
  const int64_t n_groups = ((N + 15) / 16 + c.NT - 1) / c.NT;
  const int64_t m_groups = (M + 16 * c.MT - 1) / (16 * c.MT);
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = dispatch_fmt<false, false>(w_fmt, c, dim3((unsigned)n_groups, (unsigned)m_groups, 2), p, s);
  if (e != hipSuccess) {
    set_error("mxl_mx_gemm_dual: launch failed: %s", hipGetErrorString(e));
    return MXL_EHIP;
  }
  e = launch_splitk_reduce((const float*)workspace, (const uint16_t*)bias, (uint16_t*)out, M, N, ldc, 2, s, 1.0f,
                           kOutBf16);
  if (e != hipSuccess) {
    set_error("mxl_mx_gemm_dual: split-K reduce launch failed: %s", hipGetErrorString(e));
    return MXL_EHIP;
  }
  return MXL_OK;
}

extern "C" int mxl_mx_gemm_dual(const void* hi, const void* s_hi, const void* res, const void* s_res, int64_t M,
                                const void* w_tiled, const void* sw_tiled, int64_t N, int64_t K, int w_fmt,
                                const void* bias, void* out, int64_t ldc, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  return gemm_dual_common(hi, s_hi, res, s_res, M, w_tiled, sw_tiled, N, K, w_fmt, bias, out, ldc, workspace,
                          workspace_bytes, GemmOptions(), stream);
}

extern "C" int mxl_mx_gemm_dual_ex(const void* hi, const void* s_hi, const void* res, const void* s_res, int64_t M,
                                   const void* w_tiled, const void* sw_tiled, int64_t N, int64_t K, int w_fmt,
                                   const void* bias, void* out, int64_t ldc, void* workspace, int64_t workspace_bytes,
                                   const void* options, void* stream) {
  return gemm_dual_common(hi, s_hi, res, s_res, M, w_tiled, sw_tiled, N, K, w_fmt, bias, out, ldc, workspace,
                          workspace_bytes, options_of(options), stream);
}

extern "C" int mxl_block_fp8_gemm(const void* a, const void* sa_colmajor, int64_t M, const void* w_tiled,
                                  const void* sb, int64_t N, int64_t K, const void* bias, void* out, int64_t ldc,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  return gemm_common(a, sa_colmajor, M, w_tiled, sb, N, K, kE4M3, true, bias, out, ldc, workspace, workspace_bytes,
                     GemmOptions(), stream, "mxl_block_fp8_gemm");
}

extern "C" int mxl_block_fp8_gemm_ex(const void* a, const void* sa_colmajor, int64_t M, const void* w_tiled,
                                     const void* sb, int64_t N, int64_t K, const void* bias, void* out, int64_t ldc,
                                     void* workspace, int64_t workspace_bytes, const void* options, void* stream) {
  return gemm_common(a, sa_colmajor, M, w_tiled, sb, N, K, kE4M3, true, bias, out, ldc, workspace, workspace_bytes,
                     options_of(options), stream, "mxl_block_fp8_gemm_ex");
}

// The fused producers run on the 16-row-unit schedule the unfused call picks below 32
// routed rows per expert (when the unit's operands fit in LDS); 0 otherwise.  Measured
// on the MoE layer (256 experts, hidden 2048, I 512): at 128 tokens the fused kernels
// cost what the producer and the GEMM cost apart (w2 with SwiGLU 53.3 us against 50.2 +
// 2.9) and save two launches; at 2048 tokens (96-row units, four waves per CU) the
// SwiGLU inside the GEMM took 107.4 us against 74.6 + 12.9 apart, since the standalone
// producer spreads its exp and divide work over far more waves.
static int fused_grouped_mt(int64_t routed_rows, int64_t num_experts, int64_t K, int fmt) {
  const int mt = routed_rows < 32 * num_experts ? 1 : 0;
  return mt && stream_grouped_fused_eligible(K, num_experts, fmt, mt) ? mt : 0;
}

extern "C" int mxl_grouped_fused_supported(int64_t routed_rows, int64_t num_experts, int64_t K, int w_fmt) {
  return routed_rows > 0 && num_experts > 0 && K > 0 && K % 128 == 0 && valid_wfmt(w_fmt) &&
         fused_grouped_mt(routed_rows, num_experts, K, w_fmt) != 0;
}

static int grouped_fused(const char* who, const void* x, int64_t ldx, const int32_t* row_index, int row_div,
                         const int64_t* expert_offsets, int64_t num_experts, int64_t routed_rows, const void* w_tiled,
                         const void* sw_tiled, int64_t N, int64_t K, int w_fmt, int prod, int rule, void* out,
                         void* stream) {
  MXL_CHECK_ARG(valid_wfmt(w_fmt), "%s: unknown weight format %d", who, w_fmt);
  MXL_CHECK_ARG(rule == kFloorCarry175 || rule == kCeilDiv448 || rule == kRpUe8m0, "%s: unknown rule %d", who, rule);
  MXL_CHECK_ARG(N > 0 && K > 0 && K % 128 == 0 && num_experts > 0 && row_div >= 1 && routed_rows >= 0,
                "%s: need N > 0, K %% 128 == 0, experts > 0", who);
  MXL_CHECK_ARG(ldx % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w_tiled & 15) == 0,
                "%s: bf16 rows must be 16-byte aligned (row stride %% 8 == 0)", who);
  if (routed_rows == 0) return MXL_OK;
  const int mt = fused_grouped_mt(routed_rows, num_experts, K, w_fmt);
  if (!mt) {
    set_error("%s: no fused schedule for %lld routed rows over %lld experts at K=%lld (use the unfused calls)", who,
              (long long)routed_rows, (long long)num_experts, (long long)K);
    return MXL_EUNSUPPORTED;
  }
  GemmParams p{};
  p.a = (const uint8_t*)x; p.w = (const uint8_t*)w_tiled; p.sw = sw_tiled;
  p.out = (uint16_t*)out; p.row_index = row_index; p.expert_offsets = expert_offsets;
  p.lda = ldx; p.ldc = N; p.M = routed_rows; p.N = N; p.K = K; p.KT = (K + kTileK - 1) / kTileK;
  p.w_expert_stride = mxl_tiled_weight_bytes(N, K, w_fmt);
  p.sw_expert_stride = mxl_tiled_scale_bytes(N, K);
  p.row_div = row_div; p.S = 1;
  const hipError_t e = launch_gemm_stream_grouped(w_fmt, p, num_experts, mt, (hipStream_t)stream, prod, rule);
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", who, hipGetErrorString(e));
    return MXL_EHIP;
  }
  return MXL_OK;
}

extern "C" int mxl_grouped_gemm_quant(const void* x, int64_t ldx, const int32_t* row_index, int row_div,
                                      const int64_t* expert_offsets, int64_t num_experts, int64_t routed_rows,
                                      const void* w_tiled, const void* sw_tiled, int64_t N, int64_t K, int w_fmt,
                                      int rule, void* out, void* stream) {
  MXL_CHECK_ARG(ldx >= K, "mxl_grouped_gemm_quant: row stride < K");
  return grouped_fused("mxl_grouped_gemm_quant", x, ldx, row_index, row_div, expert_offsets, num_experts, routed_rows,
                       w_tiled, sw_tiled, N, K, w_fmt, 1, rule, out, stream);
}

extern "C" int mxl_grouped_gemm_swiglu(const void* gate_up, const int64_t* expert_offsets, int64_t num_experts,
                                       int64_t routed_rows, const void* w_tiled, const void* sw_tiled, int64_t N,
                                       int64_t K, int w_fmt, int rule, void* out, void* stream) {
  return grouped_fused("mxl_grouped_gemm_swiglu", gate_up, 2 * K, nullptr, 1, expert_offsets, num_experts,
                       routed_rows, w_tiled, sw_tiled, N, K, w_fmt, 2, rule, out, stream);
}

static int grouped_common(const void* a, const void* sa, int64_t a_rows, const int32_t* row_index, int row_div,
                          const int64_t* expert_offsets, int64_t num_experts, int64_t routed_rows,
                          const void* w_tiled, const void* sw_tiled, int64_t N, int64_t K, int w_fmt, void* out,
                          const GemmOptions& o, void* stream);

// ------------------------------------------------ down projection + weighted combine

// Same layout as mxl_moe_combine in include/mxlinear.h.
struct MoeCombine {
  const int32_t* sorted_routes;
  const int32_t* inverse;
  const float* topk_weights;
  int64_t T, topk;
  void* out;
  int32_t* counters;
};

// The 16-row or 96-row weight-streaming schedule of a down projection whose combine runs
// in the kernel (prod 0: MXFP8 operands; prod 2: the SwiGLU producer, 16-row units
// only); 0 when the shape takes another schedule.
static int combine_grouped_mt(int64_t routed_rows, int64_t num_experts, int64_t K, int fmt, int prod) {
  if (K > kTileK) return 0;  // one super-tile per wave: the whole-line (coherent) store path
  if (prod == 2) return fused_grouped_mt(routed_rows, num_experts, K, fmt);
  if (prod != 0) return 0;
  // the 16-row units (below 32 routed rows per expert): the small-batch schedule
  return routed_rows < 32 * num_experts && stream_grouped_eligible(K, num_experts, fmt, 1) ? 1 : 0;
}

extern "C" int mxl_grouped_combine_supported(int64_t routed_rows, int64_t num_experts, int64_t N, int64_t K,
                                             int w_fmt, int prod) {
  return routed_rows > 0 && num_experts > 0 && N > 0 && N % 8 == 0 && K > 0 && K % 128 == 0 && valid_wfmt(w_fmt) &&
         (prod == 0 || prod == 2) && combine_grouped_mt(routed_rows, num_experts, K, w_fmt, prod) != 0;
}

static int grouped_combine_common(const char* who, const void* a, const void* sa, int64_t a_rows,
                                  const int32_t* row_index, int row_div, const int64_t* expert_offsets,
                                  int64_t num_experts, int64_t routed_rows, const void* w_tiled, const void* sw_tiled,
                                  int64_t N, int64_t K, int w_fmt, int prod, int rule, void* routed_out,
                                  const void* combine, void* stream) {
  MXL_CHECK_ARG(valid_wfmt(w_fmt), "%s: unknown weight format %d", who, w_fmt);
  MXL_CHECK_ARG(prod == 0 || rule == kCeilDiv448 || rule == kRpUe8m0, "%s: unknown SwiGLU rule %d", who, rule);
  MXL_CHECK_ARG(N > 0 && N % 8 == 0 && K > 0 && K % 128 == 0 && num_experts > 0 && routed_rows >= 0 && row_div >= 1,
                "%s: need N %% 8 == 0, K %% 128 == 0, experts > 0", who);
  MXL_CHECK_ARG(combine != nullptr, "%s: no combine descriptor", who);
  const MoeCombine c = *static_cast<const MoeCombine*>(combine);
  MXL_CHECK_ARG(c.T >= 0 && c.topk >= 1 && c.topk <= 16 && routed_rows <= c.T * c.topk,
                "%s: need 1 <= topk <= 16 and routed rows <= T * topk", who);
  MXL_CHECK_ARG(routed_rows * N * 2 < (int64_t(1) << 31), "%s: the routed output must stay below 2 GiB", who);
  MXL_CHECK_ARG(c.out && c.counters && c.inverse && c.topk_weights && (routed_rows == 0 || c.sorted_routes),
                "%s: combine descriptor has a null pointer", who);
  MXL_CHECK_ARG(((uintptr_t)a & 15) == 0 && ((uintptr_t)w_tiled & 15) == 0 && ((uintptr_t)routed_out & 15) == 0 &&
                    ((uintptr_t)c.out & 15) == 0,
                "%s: operands and outputs must be 16-byte aligned", who);
  if (c.T == 0) return MXL_OK;
  const int mt = combine_grouped_mt(routed_rows > 0 ? routed_rows : 1, num_experts, K, w_fmt, prod);
  if (!mt) {
    set_error("%s: no weight-streaming schedule for %lld routed rows over %lld experts at K=%lld", who,
              (long long)routed_rows, (long long)num_experts, (long long)K);
    return MXL_EUNSUPPORTED;
  }
  GemmParams p{};
  p.a = (const uint8_t*)a; p.sa = sa; p.w = (const uint8_t*)w_tiled; p.sw = sw_tiled;
  p.out = (uint16_t*)routed_out; p.row_index = row_index; p.expert_offsets = expert_offsets;
  p.lda = prod ? 2 * K : K; p.ldc = N; p.M = routed_rows; p.N = N; p.K = K; p.KT = (K + kTileK - 1) / kTileK;
  p.a_rows = a_rows;
  p.w_expert_stride = mxl_tiled_weight_bytes(N, K, w_fmt);
  p.sw_expert_stride = mxl_tiled_scale_bytes(N, K);
  p.row_div = row_div; p.S = 1;
  p.comb_out = (uint16_t*)c.out; p.comb_w = c.topk_weights; p.comb_inv = c.inverse;
  p.comb_routes = c.sorted_routes; p.comb_cnt = c.counters; p.comb_T = c.T; p.comb_topk = (int)c.topk;
  const hipError_t e = launch_gemm_stream_grouped(w_fmt, p, num_experts, mt, (hipStream_t)stream, prod, rule, true);
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", who, hipGetErrorString(e));
    return MXL_EHIP;
  }
  return MXL_OK;
}

extern "C" int mxl_grouped_gemm_combine(const void* a, const void* sa, int64_t a_rows, const int32_t* row_index,
                                        int row_div, const int64_t* expert_offsets, int64_t num_experts,
                                        int64_t routed_rows, const void* w_tiled, const void* sw_tiled, int64_t N,
                                        int64_t K, int w_fmt, void* routed_out, const void* combine, void* stream) {
  return grouped_combine_common("mxl_grouped_gemm_combine", a, sa, a_rows, row_index, row_div, expert_offsets,
                                num_experts, routed_rows, w_tiled, sw_tiled, N, K, w_fmt, 0, 0, routed_out, combine,
                                stream);
}

extern "C" int mxl_grouped_gemm_swiglu_combine(const void* gate_up, const int64_t* expert_offsets,
                                               int64_t num_experts, int64_t routed_rows, const void* w_tiled,
                                               const void* sw_tiled, int64_t N, int64_t K, int w_fmt, int rule,
                                               void* routed_out, const void* combine, void* stream) {
  return grouped_combine_common("mxl_grouped_gemm_swiglu_combine", gate_up, nullptr, routed_rows, nullptr, 1,
                                expert_offsets, num_experts, routed_rows, w_tiled, sw_tiled, N, K, w_fmt, 2, rule,
                                routed_out, combine, stream);
}

// The grouped schedule a call runs (shared by the launch and the plan query).
struct GroupedPlan {
  int kernel;     // kStream (weight-streaming units of 16 stream_mt rows), kWide or kGeneric
  int stream_mt;  // 1 or kGroupedStreamWideMT with kStream
  int MT;         // kWide: 16-row tiles per block
};

static GroupedPlan plan_grouped(int64_t a_rows, int64_t num_experts, int64_t routed_rows, int64_t K, int w_fmt,
                                const GemmOptions& o) {
  const int force = o.kernel;
  int stream_mt = 0;
  if (force == kStream || force == kStreamWide) {
    stream_mt = force == kStream ? 1 : kGroupedStreamWideMT;
  } else if (force == kAuto) {
    if (routed_rows < 32 * num_experts) stream_mt = 1;
    else if (routed_rows <= 96 * num_experts && K <= kTileK) stream_mt = kGroupedStreamWideMT;
  }
  if (stream_mt && !stream_grouped_eligible(K, num_experts, w_fmt, stream_mt)) stream_mt = 0;
  const bool wide_ok = K % 256 == 0 && a_rows * K < (int64_t(1) << 32) && num_experts <= kWideGroupedMaxExperts;
  if (!stream_mt && force != kGeneric && wide_ok && (force == kWide || routed_rows >= 32 * num_experts))
    return GroupedPlan{kWide, 0, o.tile_m == 4 ? 4 : 8};
  if (stream_mt) return GroupedPlan{kStream, stream_mt, 0};
  return GroupedPlan{kGeneric, 0, 0};
}

extern "C" int mxl_grouped_gemm(const void* a, const void* sa, int64_t a_rows, const int32_t* row_index, int row_div,
                                const int64_t* expert_offsets, int64_t num_experts, int64_t routed_rows,
                                const void* w_tiled, const void* sw_tiled, int64_t N, int64_t K, int w_fmt,
                                void* out, void* stream) {
  return grouped_common(a, sa, a_rows, row_index, row_div, expert_offsets, num_experts, routed_rows, w_tiled,
                        sw_tiled, N, K, w_fmt, out, GemmOptions(), stream);
}

extern "C" int mxl_grouped_gemm_ex(const void* a, const void* sa, int64_t a_rows, const int32_t* row_index,
                                   int row_div, const int64_t* expert_offsets, int64_t num_experts,
                                   int64_t routed_rows, const void* w_tiled, const void* sw_tiled, int64_t N,
                                   int64_t K, int w_fmt, void* out, const void* options, void* stream) {
  return grouped_common(a, sa, a_rows, row_index, row_div, expert_offsets, num_experts, routed_rows, w_tiled,
                        sw_tiled, N, K, w_fmt, out, options_of(options), stream);
}

static int grouped_common(const void* a, const void* sa, int64_t a_rows, const int32_t* row_index, int row_div,
                          const int64_t* expert_offsets, int64_t num_experts, int64_t routed_rows,
                          const void* w_tiled, const void* sw_tiled, int64_t N, int64_t K, int w_fmt, void* out,
                          const GemmOptions& o, void* stream) {
  MXL_CHECK_ARG(valid_wfmt(w_fmt), "mxl_grouped_gemm: unknown weight format %d", w_fmt);
  MXL_CHECK_ARG(N > 0 && K > 0 && K % 128 == 0 && num_experts > 0 && row_div >= 1,
                "mxl_grouped_gemm: need N > 0, K %% 128 == 0, experts > 0");
  MXL_CHECK_ARG(((uintptr_t)a & 15) == 0 && ((uintptr_t)w_tiled & 15) == 0, "mxl_grouped_gemm: misaligned operands");
  if (routed_rows == 0) return MXL_OK;
  // Schedule by rows per expert: few -> weight streaming over 16-row units; up to 96 on
  // average with K one super-tile (the MoE down projection) -> weight streaming over 96-row
  // units, one per expert (each expert's weights read once); otherwise the wide kernel's
  // 128-row tiles.  (With K split over waves the many-row units run one 16-column n-tile
  // per round and measured 274 against the wide kernel's 143 us at c5's gate_up.)
  // options.kernel (tuning runs and tests): kStream forces the 16-row units, kStreamWide the
  // many-row units (where they apply), kGeneric the per-expert kernel, kWide the wide kernel.
  MXL_CHECK_ARG(o.kernel >= kAuto && o.kernel <= kStreamWide, "mxl_grouped_gemm: unknown kernel %d", o.kernel);
  MXL_CHECK_ARG(o.sa_layout == 0, "mxl_grouped_gemm: grouped activations take logical scales");
  if (!options_valid(o, "mxl_grouped_gemm")) return MXL_EINVAL;
  MXL_CHECK_ARG(default_epilogue(o), "mxl_grouped_gemm: bf16 output without scaling only");
  const GroupedPlan gp = plan_grouped(a_rows, num_experts, routed_rows, K, w_fmt, o);
  const int stream_mt = gp.stream_mt;
  if (gp.kernel == kWide) {
    // enough rows per expert on average for 128-row blocks: the wide kernel
    GemmParams p{};
    p.a = (const uint8_t*)a; p.sa = sa; p.w = (const uint8_t*)w_tiled; p.sw = sw_tiled;
    p.out = (uint16_t*)out; p.row_index = row_index; p.expert_offsets = expert_offsets;
    p.lda = K; p.ldc = N; p.M = routed_rows; p.N = N; p.K = K; p.KT = (K + kTileK - 1) / kTileK; p.a_rows = a_rows;
    p.w_expert_stride = mxl_tiled_weight_bytes(N, K, w_fmt);
    p.sw_expert_stride = mxl_tiled_scale_bytes(N, K);
    p.row_div = row_div; p.S = 1;
    WideConfig wc{2, 1, (K + kTileK - 1) / kTileK};
    // 128-row blocks: with 64 rows per expert on average (c5, T = 2048) 64-row blocks
    // measured 8-10 % slower, since experts past 64 rows then copy their weights twice
    wc.MT = gp.MT;
    hipError_t e = launch_gemm_wide(w_fmt, false, wc, p, num_experts, (hipStream_t)stream);
    if (e != hipSuccess) {
      set_error("mxl_grouped_gemm: launch failed: %s", hipGetErrorString(e));
      return MXL_EHIP;
    }
    return MXL_OK;
  }
  if (stream_mt) {
    // persistent workgroups stream each expert's weights past its rows
    GemmParams p{};
    p.a = (const uint8_t*)a; p.sa = sa; p.w = (const uint8_t*)w_tiled; p.sw = sw_tiled;
    p.out = (uint16_t*)out; p.row_index = row_index; p.expert_offsets = expert_offsets;
    p.lda = K; p.ldc = N; p.M = routed_rows; p.N = N; p.K = K; p.KT = (K + kTileK - 1) / kTileK; p.a_rows = a_rows;
    p.w_expert_stride = mxl_tiled_weight_bytes(N, K, w_fmt);
    p.sw_expert_stride = mxl_tiled_scale_bytes(N, K);
    p.row_div = row_div; p.S = 1;
    hipError_t e = launch_gemm_stream_grouped(w_fmt, p, num_experts, stream_mt, (hipStream_t)stream);
    if (e != hipSuccess) {
      set_error("mxl_grouped_gemm: launch failed: %s", hipGetErrorString(e));
      return MXL_EHIP;
    }
    return MXL_OK;
  }
  GemmConfig c;
  const int64_t KT = (K + kTileK - 1) / kTileK;
  c.MT = 1; c.NT = 1; c.S = 1;
  c.KW = (int)(KT >= 4 ? 4 : KT);
  GemmParams p{};
  p.a = (const uint8_t*)a; p.sa = sa; p.w = (const uint8_t*)w_tiled; p.sw = sw_tiled;
  p.out = (uint16_t*)out; p.row_index = row_index; p.expert_offsets = expert_offsets;
  p.lda = K; p.ldc = N; p.M = routed_rows; p.N = N; p.K = K; p.KT = KT; p.a_rows = a_rows;
  p.w_expert_stride = mxl_tiled_weight_bytes(N, K, w_fmt);
  p.sw_expert_stride = mxl_tiled_scale_bytes(N, K);
  p.row_div = row_div; p.S = 1;
  dim3 grid((unsigned)((N + 15) / 16), (unsigned)num_experts, 1);
  hipError_t e = dispatch_fmt<false, true>(w_fmt, c, grid, p, (hipStream_t)stream);
  if (e != hipSuccess) {
    set_error("mxl_grouped_gemm: launch failed: %s", hipGetErrorString(e));
    return MXL_EHIP;
  }
  return MXL_OK;
}

// ------------------------------------------------------------------ plan names

// The kernels a call launches, named as the profiler prints them (template arguments
// without spaces), joined by " + ".  For matching profiles to the code that runs.
static int plan_name_out(const std::string& name, char* buf, int64_t len) {
  MXL_CHECK_ARG(buf && len > (int64_t)name.size(), "plan name needs %lld bytes", (long long)name.size() + 1);
  memcpy(buf, name.c_str(), name.size() + 1);
  return MXL_OK;
}

static const char* tf(bool b) { return b ? "true" : "false"; }

extern "C" int mxl_gemm_plan_name(int64_t M, int64_t N, int64_t K, int w_fmt, int block, const void* options,
                                  char* buf, int64_t len) {
  MXL_CHECK_ARG(M > 0 && N > 0 && K > 0 && K % 128 == 0 && valid_wfmt(w_fmt), "mxl_gemm_plan_name: bad shape");
  const GemmOptions o = options_of(options);
  if (!options_valid(o, "mxl_gemm_plan_name")) return MXL_EINVAL;
  DensePlan d;
  if (!plan_dense(M, N, K, w_fmt, block != 0, o, d)) {
    set_error("mxl_gemm_plan_name: kernel %d does not run this shape", o.kernel);
    return MXL_EUNSUPPORTED;
  }
  char k[160];
  std::string name;
  const int64_t KT = (K + kTileK - 1) / kTileK;
  int S = 1;
  if (d.kernel == kStream) {
    const bool db = KT <= stream_max_waves(block != 0);
    snprintf(k, sizeof k, "gemm_stream_kernel<%d,%d,%s,%s,-1,-1>", w_fmt, db ? 1 : 2, tf(db), tf(block != 0));
    name = k;
  } else if (d.kernel == kChunk) {
    snprintf(k, sizeof k, "gemm_chunk_kernel<%d,%d,1>", w_fmt, kChunkSuperTiles);
    name = k;
    S = (int)chunk_count(K, kChunkSuperTiles);
  } else if (d.kernel == kWide) {
    snprintf(k, sizeof k, "gemm_wide_kernel<%d,%d,%d,%s,false,%d>", w_fmt, d.wide.MT, d.wide.NT, tf(block != 0),
             d.wide.WM);
    name = k;
    if (d.wide.dp_tiles > 0 || d.wide.S > 1) name += " + wide_tile_reduce_kernel";
    S = 1;  // (its split reduce is the tile reduce)
  } else {
    snprintf(k, sizeof k, "gemm_kernel<%d,%d,%d,%s,false>", w_fmt, d.gen.MT, d.gen.NT, tf(block != 0));
    name = k;
    S = d.gen.S;
  }
  if (S > 1) name += N % 8 == 0 ? " + splitk_reduce8_kernel" : " + splitk_reduce_kernel";
  return plan_name_out(name, buf, len);
}

extern "C" int mxl_grouped_plan_name(int64_t routed_rows, int64_t num_experts, int64_t K, int w_fmt, int prod,
                                     int rule, const void* options, char* buf, int64_t len) {
  MXL_CHECK_ARG(routed_rows > 0 && num_experts > 0 && K > 0 && K % 128 == 0 && valid_wfmt(w_fmt) && prod >= 0 &&
                    prod <= 2,
                "mxl_grouped_plan_name: bad shape");
  const GemmOptions o = options_of(options);
  if (!options_valid(o, "mxl_grouped_plan_name")) return MXL_EINVAL;
  char k[160];
  if (prod) {  // the fused producers run the 16-row units
    snprintf(k, sizeof k, "gemm_stream_grouped_kernel<%d,1,%d>", w_fmt, 4 * prod + rule);
    return plan_name_out(k, buf, len);
  }
  const GroupedPlan gp = plan_grouped(routed_rows, num_experts, routed_rows, K, w_fmt, o);
  if (gp.kernel == kWide)
    snprintf(k, sizeof k, "gemm_wide_kernel<%d,%d,2,false,true,1>", w_fmt, gp.MT);
  else if (gp.kernel == kStream)
    snprintf(k, sizeof k, "gemm_stream_grouped_kernel<%d,%d,0>", w_fmt, gp.stream_mt);
  else
    snprintf(k, sizeof k, "gemm_kernel<%d,1,1,false,true>", w_fmt);
  return plan_name_out(k, buf, len);
}
