// LDS-staged MX GEMM for prefill-sized M on gfx950.
//
// Workgroup tile 128 (M) x 128 (N), four wavefronts in a 2 x 2 grid, each
// owning 64 x 64 = 4 x 4 MFMA tiles of 16 x 16.  K advances in steps of 256
// (half of a 512-wide weight super-tile), double-buffered in LDS:
//
//   A (row-major activations) is scattered on the way in so that the LDS image
//     is in MFMA fragment order: m-tile mt, piece g = 2 jj + half holds, at
//     lane l = 16q + r, the 16 bytes K [128 jj + 64 half + 16 q, +16) of row
//     16 mt + r.  Wave w copies m-tiles 2w and 2w+1: lane l reads 64
//     contiguous bytes per row across 4 lanes and writes 1 KiB contiguous, so
//     both the global read and the LDS write are conflict-free.
//   B (weights) is copied verbatim from the MFMA-tiled layout: the half
//     super-tile of each n-tile is contiguous (4 KiB E4M3, 3 KiB FP6).
//
// Each step: issue the next step's global loads, run 2 x 16 MFMAs per wave
// from LDS (fragment reads are lane-contiguous 16-byte loads), write the
// staged registers into the other LDS buffer, one barrier.  E8M0 scales are
// read per wave straight from global memory (row-major activation scales,
// tiled weight scales), one step ahead.  When the tile grid cannot cover the
// GPU, S workgroups split K and write fp32 partials reduced in split order.
#include "gemm_common.h"

namespace mxl {

constexpr int kBM = 128, kBN = 128;

template <int FMT>
struct LdsCfg {
  static constexpr int CH = FmtTraits<FMT>::CH;
  static constexpr int BCH = CH / 2;                 // 1 KiB B chunks per n-tile per step
  static constexpr int A_BYTES = (kBM / 16) * 4 * 1024;
  static constexpr int B_BYTES = (kBN / 16) * BCH * 1024;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int B_LOADS = (kBN / 16) * BCH * 64 / 256;  // 16-byte pieces per thread
};

struct StepScales {
  uint32_t a[4][2];  // byte q of the activation scale dword, per m-tile and MFMA of the step
  uint32_t b[4];     // tiled weight scale dword per n-tile (byte j = MFMA j)
};

template <int FMT, int J>
__device__ __forceinline__ void mfma_tile(const v8i (&af)[4], const v8i (&bf)[4], const StepScales& sc, int jj,
                                          v4f (&acc)[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = mfma_step<FMT, J>(af[i], bf[n], acc[i][n], sc.a[i][jj], sc.b[n]);
}

template <int FMT>
__device__ __forceinline__ void lds_load_step(const GemmParams& p, int64_t st, int t, int lane, int q, int64_t nt0,
                                              int64_t ntiles_total, const int64_t (&copy_row)[2],
                                              const int64_t (&frag_row)[4], const int64_t (&ntile_ld)[4],
                                              uint4 (&ra)[8], uint4 (&rb)[LdsCfg<FMT>::B_LOADS],
                                              StepScales& sc) {
  using C = LdsCfg<FMT>;
  const int64_t kt = st >> 1, h = st & 1;
  const int64_t kbase = kt * kTileK + 256 * h;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int g = i & 3;
    const int64_t k = kbase + 64 * g + 16 * q;
    ra[i] = k < p.K ? *reinterpret_cast<const uint4*>(p.a + copy_row[i >> 2] * p.lda + k) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < C::B_LOADS; ++i) {
    const int piece = i * 256 + t;
    const int nt = piece / (C::BCH * 64), off = piece % (C::BCH * 64);
    int64_t ntile = nt0 + nt;
    if (ntile >= ntiles_total) ntile = ntiles_total - 1;
    rb[i] = *reinterpret_cast<const uint4*>(p.w + (ntile * p.KT + kt) * (C::CH * 1024) + h * (C::BCH * 1024) + off * 16);
  }
  const uint8_t* sa_base = static_cast<const uint8_t*>(p.sa);
  const uint8_t* sw_base = static_cast<const uint8_t*>(p.sw);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int64_t kb = kt * 16 + 4 * (2 * h + jj);
      uint32_t v = 0;
      if (kb * 32 < p.K) v = *reinterpret_cast<const uint32_t*>(sa_base + frag_row[i] * (p.K / 32) + kb);
      sc.a[i][jj] = (v >> (8 * q)) & 0xFFu;
    }
#pragma unroll
  for (int n = 0; n < 4; ++n)
    sc.b[n] = *reinterpret_cast<const uint32_t*>(sw_base + (ntile_ld[n] * p.KT + kt) * 256 + lane * 4);
}

template <int FMT>
__device__ __forceinline__ void lds_store_step(uint8_t* L, int t, int lane, int wv, const uint4 (&ra)[8],
                                               const uint4 (&rb)[LdsCfg<FMT>::B_LOADS]) {
  using C = LdsCfg<FMT>;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int mt = 2 * wv + (i >> 2), g = i & 3;
    *reinterpret_cast<uint4*>(L + (mt * 4 + g) * 1024 + lane * 16) = ra[i];
  }
#pragma unroll
  for (int i = 0; i < C::B_LOADS; ++i) *reinterpret_cast<uint4*>(L + C::A_BYTES + (i * 256 + t) * 16) = rb[i];
}

template <int FMT>
__global__ __launch_bounds__(256) void gemm_lds_kernel(GemmParams p, int steps_per_split) {
  using C = LdsCfg<FMT>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][C::STAGE];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int wm = wv >> 1, wn = wv & 1;
  const int64_t row0 = (int64_t)blockIdx.y * kBM;
  const int64_t nt0 = (int64_t)blockIdx.x * (kBN / 16);
  const int64_t ntiles_total = (p.N + 15) / 16;
  const int64_t split = blockIdx.z;
  const int64_t total_steps = 2 * p.KT;
  const int64_t s_begin = split * steps_per_split;
  const int64_t s_end = s_begin + steps_per_split < total_steps ? s_begin + steps_per_split : total_steps;
  // rows this thread copies (A staging) and rows its fragments cover (scales)
  int64_t copy_row[2], frag_row[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int64_t row = row0 + (2 * wv + i) * 16 + r;
    copy_row[i] = row < p.M ? row : p.M - 1;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = row0 + (wm * 4 + i) * 16 + r;
    frag_row[i] = row < p.M ? row : p.M - 1;
  }
  int64_t ntile_ld[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int64_t nt = nt0 + wn * 4 + n;
    ntile_ld[n] = nt < ntiles_total ? nt : ntiles_total - 1;
  }

  uint4 ra[8], rb[C::B_LOADS];
  StepScales sc_next, sc_cur;
  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = v4f{0.f, 0.f, 0.f, 0.f};

  if (s_begin < s_end) {
    lds_load_step<FMT>(p, s_begin, t, lane, q, nt0, ntiles_total, copy_row, frag_row, ntile_ld, ra, rb, sc_next);
    lds_store_step<FMT>(lds[0], t, lane, wv, ra, rb);
    sc_cur = sc_next;
    __syncthreads();
    for (int64_t st = s_begin; st < s_end; ++st) {
      const int buf = (int)((st - s_begin) & 1);
      if (st + 1 < s_end)
        lds_load_step<FMT>(p, st + 1, t, lane, q, nt0, ntiles_total, copy_row, frag_row, ntile_ld, ra, rb, sc_next);
      const uint8_t* L = lds[buf];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        v8i af[4], bf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint8_t* base = L + ((wm * 4 + i) * 4 + 2 * jj) * 1024 + lane * 16;
          const uint4 lo = *reinterpret_cast<const uint4*>(base);
          const uint4 hi = *reinterpret_cast<const uint4*>(base + 1024);
          af[i] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const uint8_t* base = L + C::A_BYTES + (wn * 4 + n) * (C::BCH * 1024) + lane * 16;
          if (FMT == kE4M3) {
            const uint4 lo = *reinterpret_cast<const uint4*>(base + 2 * jj * 1024);
            const uint4 hi = *reinterpret_cast<const uint4*>(base + (2 * jj + 1) * 1024);
            bf[n] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
          } else {
            // the lane's 12 dwords of this step; MFMA jj takes dwords [6jj, 6jj + 6)
            if (jj == 0) {
              const uint4 c0 = *reinterpret_cast<const uint4*>(base);
              const uint2 c1 = *reinterpret_cast<const uint2*>(base + 1024);
              bf[n] = v8i{(int)c0.x, (int)c0.y, (int)c0.z, (int)c0.w, (int)c1.x, (int)c1.y, 0, 0};
            } else {
              const uint2 c1 = *reinterpret_cast<const uint2*>(base + 1024 + 8);
              const uint4 c2 = *reinterpret_cast<const uint4*>(base + 2048);
              bf[n] = v8i{(int)c1.x, (int)c1.y, (int)c2.x, (int)c2.y, (int)c2.z, (int)c2.w, 0, 0};
            }
          }
        }
        const bool h1 = (st & 1) != 0;
        if (jj == 0) {
          if (h1) mfma_tile<FMT, 2>(af, bf, sc_cur, 0, acc); else mfma_tile<FMT, 0>(af, bf, sc_cur, 0, acc);
        } else {
          if (h1) mfma_tile<FMT, 3>(af, bf, sc_cur, 1, acc); else mfma_tile<FMT, 1>(af, bf, sc_cur, 1, acc);
        }
      }
      if (st + 1 < s_end) {
        lds_store_step<FMT>(lds[buf ^ 1], t, lane, wv, ra, rb);
        sc_cur = sc_next;
      }
      __syncthreads();
    }
  }

  // epilogue: lane holds rows 4q + e, column r of each 16 x 16 tile
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int64_t nt = nt0 + wn * 4 + n;
      const int64_t col = nt * 16 + r;
      if (nt >= ntiles_total || col >= p.N) continue;
      const float bias = p.bias ? bf16_to_f32(p.bias[col]) : 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t row = row0 + (wm * 4 + i) * 16 + 4 * q + e;
        if (row >= p.M) continue;
        if (p.S > 1) {
          p.partial[(split * p.M + row) * p.N + col] = acc[i][n][e];
        } else {
          float y = bf16_round(acc[i][n][e]);
          if (p.bias) y = y + bias;
          p.out[row * p.ldc + col] = f32_to_bf16(y);
        }
      }
    }
}

bool lds_gemm_eligible(int64_t M, int64_t N, int64_t K, int fmt, bool block) {
  return !block && M >= 64 && (fmt == kE4M3 || fmt == kE2M3 || fmt == kE3M2);
}

// K splits so that the tile grid covers the 256 CUs; every split gets >= 2 steps.
int lds_gemm_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  const int64_t steps = 2 * ((K + kTileK - 1) / kTileK);
  int64_t S = 1;
  if (tiles < 192) {
    S = (256 + tiles - 1) / tiles;
    if (S > steps / 2) S = steps / 2;
    if (S < 1) S = 1;
  }
  return (int)S;
}

hipError_t launch_gemm_lds(int fmt, const GemmParams& p, int S, hipStream_t stream) {
  const int64_t steps = 2 * p.KT;
  const int steps_per_split = (int)((steps + S - 1) / S);
  dim3 grid((unsigned)((p.N + kBN - 1) / kBN), (unsigned)((p.M + kBM - 1) / kBM), (unsigned)S);
  if (fmt == kE4M3) hipLaunchKernelGGL(gemm_lds_kernel<kE4M3>, grid, dim3(256), 0, stream, p, steps_per_split);
  else if (fmt == kE2M3) hipLaunchKernelGGL(gemm_lds_kernel<kE2M3>, grid, dim3(256), 0, stream, p, steps_per_split);
  else if (fmt == kE3M2) hipLaunchKernelGGL(gemm_lds_kernel<kE3M2>, grid, dim3(256), 0, stream, p, steps_per_split);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace mxl
