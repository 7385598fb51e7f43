// LDS-staged MX GEMM for prefill-sized M on gfx950.
//
// Workgroup tile 128 (M) x 128 (N), four wavefronts in a 2 x 2 grid, each
// owning 64 x 64 = 4 x 4 MFMA tiles of 16 x 16.  K advances in stages of 256
// (half of a 512-wide weight super-tile), double-buffered in LDS, filled by
// direct global->LDS loads (global_load_lds_dwordx4: lane i of a wave writes
// 16 bytes at LDS base + 16 i, no staging registers):
//
//   A (row-major activations): the LDS image is in MFMA fragment order.
//     Piece g = 2 jj + half of m-tile mt holds, at lane l = 16q + r, the 16
//     bytes K [128 jj + 64 half + 16 q, +16) of row 16 mt + r -- so the wave
//     that copies (mt, g) reads 64 contiguous bytes per row (4 lanes) and the
//     DMA writes 1 KiB contiguous.  Wave w copies m-tiles 2w and 2w + 1.
//   B (weights): the half super-tile of each n-tile is contiguous in the
//     MFMA-tiled layout (4 KiB E4M3, 3 KiB FP6) and is copied verbatim.
//
// A loop iteration covers one super-tile (two stages), so the MFMA op_sel
// immediates (which byte of each E8M0 dword) are static.  Per stage: start the
// next stage's DMA, run 2 x 16 MFMAs per wave from lane-contiguous LDS
// fragment reads, wait for the DMA, one barrier.  E8M0 scales come straight
// from global memory one super-tile ahead (a 16-byte load per m-tile row of
// activation scales, a dword per n-tile of tiled weight scales).  When the tile
// grid cannot cover the GPU, S workgroups split K on super-tile boundaries
// and write fp32 partials that a second kernel reduces in split order.
#include "gemm_common.h"

namespace mxl {

constexpr int kBM = 128, kBN = 128;

template <int FMT>
struct LdsCfg {
  static constexpr int CH = FmtTraits<FMT>::CH;
  static constexpr int BCH = CH / 2;  // 1 KiB B chunks per n-tile per stage
  static constexpr int A_BYTES = (kBM / 16) * 4 * 1024;
  static constexpr int B_BYTES = (kBN / 16) * BCH * 1024;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int B_WAVE_COPIES = (kBN / 16) * BCH / 4;  // 1 KiB copies per wave
};

typedef __attribute__((address_space(1))) const void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;

__device__ __forceinline__ void dma16(const void* src, uint8_t* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((gptr_t)src, (lptr_t)lds_wave_base, 16, 0, 0);
}

struct SuperScales {
  uint4 a[4];     // activation E8M0 bytes of blocks 16kt .. 16kt+15 of each fragment row
  uint32_t b[4];  // tiled weight scale dword per n-tile (byte j = MFMA j)
};

// DMA one stage (super-tile kt, half h) into LDS buffer L.
template <int FMT>
__device__ __forceinline__ void stage_copy(const GemmParams& p, uint8_t* L, int64_t kt, int h, int wv, int lane,
                                           int q, int64_t nt0, int64_t ntiles_total,
                                           const int64_t (&copy_row)[2]) {
  using C = LdsCfg<FMT>;
  const int64_t kbase = kt * kTileK + 256 * h;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int mt = 2 * wv + (i >> 2), g = i & 3;
    dma16(p.a + copy_row[i >> 2] * p.lda + kbase + 64 * g + 16 * q, L + (mt * 4 + g) * 1024);
  }
#pragma unroll
  for (int i = 0; i < C::B_WAVE_COPIES; ++i) {
    const int piece = (i * 4 + wv) * 64 + lane;  // 16-byte piece of the stage's B image
    const int nt = piece / (C::BCH * 64), off = piece % (C::BCH * 64);
    int64_t ntile = nt0 + nt;
    if (ntile >= ntiles_total) ntile = ntiles_total - 1;
    dma16(p.w + (ntile * p.KT + kt) * (C::CH * 1024) + h * (C::BCH * 1024) + off * 16,
          L + C::A_BYTES + (i * 4 + wv) * 1024);
  }
}

__device__ __forceinline__ void load_scales(const GemmParams& p, int64_t kt, int lane,
                                            const int64_t (&frag_row)[4], const int64_t (&ntile_ld)[4],
                                            SuperScales& sc) {
  const uint8_t* sa = static_cast<const uint8_t*>(p.sa);
  const uint8_t* sw = static_cast<const uint8_t*>(p.sw);
  // rows are 8-byte aligned (K % 256 == 0); a half last super-tile has 8 scale bytes
  const bool full = (kt + 1) * kTileK <= p.K;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint8_t* rowp = sa + frag_row[i] * (p.K / 32) + kt * 16;
    const uint2 lo = *reinterpret_cast<const uint2*>(rowp);
    const uint2 hi = full ? *reinterpret_cast<const uint2*>(rowp + 8) : make_uint2(0, 0);
    sc.a[i] = make_uint4(lo.x, lo.y, hi.x, hi.y);
  }
#pragma unroll
  for (int n = 0; n < 4; ++n) sc.b[n] = *reinterpret_cast<const uint32_t*>(sw + (ntile_ld[n] * p.KT + kt) * 256 + lane * 4);
}

__device__ __forceinline__ uint32_t dword_of(const uint4& v, int j) {
  return j == 0 ? v.x : (j == 1 ? v.y : (j == 2 ? v.z : v.w));
}

// 16 MFMAs of one 128-wide K slice (MFMA index J of the super-tile) from LDS
// stage L.  The four B fragments are read once; A fragments stream one m-tile
// at a time so each LDS read overlaps the previous m-tile's MFMAs and only
// 48 fragment registers are live.
template <int FMT, int J>
__device__ __forceinline__ void stage_mfma(const uint8_t* L, int wm, int wn, int lane, int q,
                                           const SuperScales& sc, v4f (&acc)[4][4]) {
  using C = LdsCfg<FMT>;
  constexpr int jj = J & 1;
  v8i bf[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const uint8_t* base = L + C::A_BYTES + (wn * 4 + n) * (C::BCH * 1024) + lane * 16;
    if (FMT == kE4M3) {
      const uint4 lo = *reinterpret_cast<const uint4*>(base + 2 * jj * 1024);
      const uint4 hi = *reinterpret_cast<const uint4*>(base + (2 * jj + 1) * 1024);
      bf[n] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    } else if (jj == 0) {  // FP6: the lane's 12 dwords of the stage; slice jj takes [6jj, 6jj + 6)
      const uint4 c0 = *reinterpret_cast<const uint4*>(base);
      const uint2 c1 = *reinterpret_cast<const uint2*>(base + 1024);
      bf[n] = v8i{(int)c0.x, (int)c0.y, (int)c0.z, (int)c0.w, (int)c1.x, (int)c1.y, 0, 0};
    } else {
      const uint2 c1 = *reinterpret_cast<const uint2*>(base + 1024 + 8);
      const uint4 c2 = *reinterpret_cast<const uint4*>(base + 2048);
      bf[n] = v8i{(int)c1.x, (int)c1.y, (int)c2.x, (int)c2.y, (int)c2.z, (int)c2.w, 0, 0};
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint8_t* base = L + ((wm * 4 + i) * 4 + 2 * jj) * 1024 + lane * 16;
    const uint4 lo = *reinterpret_cast<const uint4*>(base);
    const uint4 hi = *reinterpret_cast<const uint4*>(base + 1024);
    const v8i af = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    const uint32_t sa = (dword_of(sc.a[i], J) >> (8 * q)) & 0xFFu;
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = mfma_step<FMT, J>(af, bf[n], acc[i][n], sa, sc.b[n]);
  }
}

// The DMA writes LDS asynchronously and is counted by vmcnt: every wave drains
// its own copies before the barrier that hands the stage to all waves.
__device__ __forceinline__ void dma_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

template <int FMT>
__global__ __launch_bounds__(256) void gemm_lds_kernel(GemmParams p, int64_t kt_per_split) {
  using C = LdsCfg<FMT>;
  // two distinct objects (not one [2][...] array) so the compiler can tell the
  // DMA target stage from the stage being read and need not drain the DMA first
  __shared__ __attribute__((aligned(1024))) uint8_t lds0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t lds1[C::STAGE];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int wm = wv >> 1, wn = wv & 1;
  const int64_t row0 = (int64_t)blockIdx.y * kBM;
  const int64_t nt0 = (int64_t)blockIdx.x * (kBN / 16);
  const int64_t ntiles_total = (p.N + 15) / 16;
  const int64_t split = blockIdx.z;
  const int64_t kt_begin = split * kt_per_split;
  const int64_t kt_end = kt_begin + kt_per_split < p.KT ? kt_begin + kt_per_split : p.KT;
  // the last super-tile may hold only its first 256 columns (K % 512 == 256)
  const bool half_last = (p.K % kTileK) != 0;

  int64_t copy_row[2], frag_row[4], ntile_ld[4];
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
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int64_t nt = nt0 + wn * 4 + n;
    ntile_ld[n] = nt < ntiles_total ? nt : ntiles_total - 1;
  }

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[i][n] = v4f{0.f, 0.f, 0.f, 0.f};

  // super-tiles [kt_begin, kt_full) are whole; a K % 512 == 256 tail is peeled
  const int64_t kt_full = (half_last && kt_end == p.KT) ? kt_end - 1 : kt_end;
  if (kt_begin < kt_end) {
    SuperScales sc, sc_next;
    stage_copy<FMT>(p, lds0, kt_begin, 0, wv, lane, q, nt0, ntiles_total, copy_row);
    load_scales(p, kt_begin, lane, frag_row, ntile_ld, sc);
    dma_wait_barrier();
    for (int64_t kt = kt_begin; kt < kt_full; ++kt) {
      // stage (kt, 0) is in lds0; fetch (kt, 1) into lds1 and the next scales
      stage_copy<FMT>(p, lds1, kt, 1, wv, lane, q, nt0, ntiles_total, copy_row);
      load_scales(p, kt + 1 < p.KT ? kt + 1 : kt, lane, frag_row, ntile_ld, sc_next);
      stage_mfma<FMT, 0>(lds0, wm, wn, lane, q, sc, acc);
      stage_mfma<FMT, 1>(lds0, wm, wn, lane, q, sc, acc);
      dma_wait_barrier();
      // stage (kt, 1) is in lds1; fetch (kt + 1, 0) into lds0
      if (kt + 1 < kt_end) stage_copy<FMT>(p, lds0, kt + 1, 0, wv, lane, q, nt0, ntiles_total, copy_row);
      stage_mfma<FMT, 2>(lds1, wm, wn, lane, q, sc, acc);
      stage_mfma<FMT, 3>(lds1, wm, wn, lane, q, sc, acc);
      dma_wait_barrier();
      sc = sc_next;
    }
    if (kt_full < kt_end) {  // the half super-tile: stage (kt_full, 0) is in lds0
      stage_mfma<FMT, 0>(lds0, wm, wn, lane, q, sc, acc);
      stage_mfma<FMT, 1>(lds0, wm, wn, lane, q, sc, acc);
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
  return !block && M >= 64 && K % 256 == 0 && (fmt == kE4M3 || fmt == kE2M3 || fmt == kE3M2);
}

// K splits (on super-tile boundaries) so that the tile grid covers the 256 CUs.
int lds_gemm_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  const int64_t KT = (K + kTileK - 1) / kTileK;
  int64_t S = 1;
  if (tiles < 192) {
    S = (256 + tiles - 1) / tiles;
    if (S > KT) S = KT;
    const int64_t per = (KT + S - 1) / S;
    S = (KT + per - 1) / per;  // no empty splits
  }
  return (int)S;
}

hipError_t launch_gemm_lds(int fmt, const GemmParams& p, int S, hipStream_t stream) {
  const int64_t kt_per_split = (p.KT + S - 1) / S;
  dim3 grid((unsigned)((p.N + kBN - 1) / kBN), (unsigned)((p.M + kBM - 1) / kBM), (unsigned)S);
  if (fmt == kE4M3) hipLaunchKernelGGL(gemm_lds_kernel<kE4M3>, grid, dim3(256), 0, stream, p, kt_per_split);
  else if (fmt == kE2M3) hipLaunchKernelGGL(gemm_lds_kernel<kE2M3>, grid, dim3(256), 0, stream, p, kt_per_split);
  else if (fmt == kE3M2) hipLaunchKernelGGL(gemm_lds_kernel<kE3M2>, grid, dim3(256), 0, stream, p, kt_per_split);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace mxl
