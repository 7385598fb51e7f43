// K-chunked weight-streaming GEMM for 17..128 activation rows on gfx950 (MX weights).
//
// At these M the weights dominate the bytes (c2 M = 128: 23.6 MB of weights against
// 1.2 MB of activations), so the design streams every weight byte once from HBM and
// keeps the activations stationary:
//
//   * the K range is cut into chunks of KC 512-wide super-tiles; a work item is one
//     (chunk, 16-column n-tile) pair, items are numbered chunk-major and split evenly
//     over at most one workgroup per CU;
//   * a workgroup has eight wavefronts, wave w owning m-tile w (rows 16 w .. 16 w + 15):
//     it holds the MFMA fragments of its rows for the whole chunk in registers (loaded
//     row-major, 64-byte spans per four lanes, and handed to the fragment lanes by
//     ds_bpermute, as the decode kernel does), so no activation byte passes through LDS;
//   * each item's weight tile (KC super-tiles of the MFMA-tiled layout, copied verbatim)
//     and its E8M0 scale dwords go global -> LDS by direct copies into a ring of R slots,
//     R - 1 items ahead; all eight waves read the tile's fragments from LDS;
//   * each wave accumulates its 16 x 16 block over the chunk in one fp32 accumulator (the
//     MFMA chain runs over the chunk's K128 slices in order) and stores it as the chunk's
//     fp32 partial ([chunk][M][N], summed in chunk order by the split-K reduce) or, with one
//     chunk, as the output element.
//
// The copies are issued from inline assembly and waited for with explicit vmcnt counts
// (vector loads complete in issue order); the activation loads are the compiler's own and
// precede the copies of the items that use them.
#include "gemm_common.h"

#pragma clang diagnostic ignored "-Winline-asm"

namespace mxl {

namespace {

typedef __attribute__((address_space(3))) uint8_t lds_u8_c;
__device__ __forceinline__ uint32_t lds_addr_c(const uint8_t* p) { return (uint32_t)(uintptr_t)(const lds_u8_c*)p; }

// Lane i copies 16 (4) bytes from base + voff to LDS [lds + 16 i] ([lds + 4 i]); base and
// lds are wave-uniform.
__device__ __forceinline__ void chunk_copy16(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(base)
               : "memory", "m0");
}
__device__ __forceinline__ void chunk_copy4(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(voff), "s"(base)
               : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void chunk_wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt immediate");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

constexpr int kChunkSlots = 4;

template <int FMT, int KC, int W>
struct ChunkSlot {
  static constexpr int CH = FmtTraits<FMT>::CH;      // 1 KiB chunks per super-tile
  static constexpr int B = 0;                         // KC x CH KiB of weight codes
  static constexpr int SB = KC * CH * 1024;           // KC x 256 B of E8M0 dwords
  static constexpr int BYTES = SB + KC * 256;
  static constexpr int NCH = KC * CH;                 // chunk copies per item
  static_assert(NCH % W == 0 && KC <= W, "the copies split evenly over the waves");
  static constexpr int CPW = NCH / W;                 // chunk copies per wave per item
  // copies per wave per item: its chunk copies, plus one scale dword copy for waves < KC
  static constexpr int C_SCALE = CPW + 1, C_PLAIN = CPW;
};

// Copy item (chunk c, n-tile nt)'s weights into a slot: wave w copies chunks w, w + W, ...
// of the item's KC x CH, and waves w < KC the scale dwords of super-tile w.
template <int FMT, int KC, int W>
__device__ __forceinline__ void chunk_copy_item(const GemmParams& p, uint8_t* slot, int64_t c, int64_t nt, int wv,
                                                int lane) {
  using S = ChunkSlot<FMT, KC, W>;
  const int64_t kt0 = c * KC;
  const uint8_t* w = p.w + (nt * p.KT + kt0) * (S::CH * 1024);
#pragma unroll
  for (int i = 0; i < S::CPW; ++i) {
    const int ch = wv + i * W;  // chunk index inside the item: super-tile ch / CH
    // super-tiles past K (a short last chunk) copy the item's first super-tile again: never read
    const int64_t u = ch / S::CH;
    const int64_t off = kt0 + u < p.KT ? (int64_t)ch * 1024 : (int64_t)(ch % S::CH) * 1024;
    chunk_copy16(w + off, (uint32_t)(lane * 16), lds_addr_c(slot + S::B + ch * 1024));
  }
  if (wv < KC) {
    const int64_t kt = kt0 + wv < p.KT ? kt0 + wv : kt0;
    chunk_copy4(static_cast<const uint8_t*>(p.sw) + (nt * p.KT + kt) * 256, (uint32_t)(lane * 4),
                lds_addr_c(slot + S::SB + wv * 256));
  }
}

template <int C, int L>
__device__ __forceinline__ void chunk_wait(int later) {
  if constexpr (L == 0) {
    chunk_wait_vm<0>();
  } else {
    if (later >= L) chunk_wait_vm<L * C>();
    else chunk_wait<C, L - 1>(later);
  }
}

}  // namespace

struct ChunkGrid {
  int64_t nchunks, ntiles, items;
};

// MTW m-tiles per wave (eight m-tiles over 8 / MTW waves).  Only MTW = 1 is launched: with
// two (four waves, each B fragment read feeding two MFMAs) c2 M = 128 took 28.6 against
// 22.2 us, and chunks of two super-tiles 23.8 us.
template <int FMT, int KC, int MTW>
__global__ __launch_bounds__(64 * (8 / MTW), 1) void gemm_chunk_kernel(GemmParams p, ChunkGrid g) {
  constexpr int W = 8 / MTW;
  using S = ChunkSlot<FMT, KC, W>;
  constexpr int R = kChunkSlots;
  constexpr int HELD = MTW == 1 ? 8 : 4;  // items whose outputs a wave holds before storing them
  __shared__ __attribute__((aligned(16))) uint8_t ring[R * S::BYTES];
  const int t = threadIdx.x, lane = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int64_t G = gridDim.x, gi = blockIdx.x;
  const int64_t i0 = gi * g.items / G, i1 = (gi + 1) * g.items / G;
  if (i0 >= i1) return;
  const bool scale_wave = wv < KC;

  // this wave's activation fragments of the current chunk (m-tiles MTW wv ..), slices past
  // K zero; the E8M0 bytes of the four slices of a super-tile packed in one dword (byte j:
  // slice j, picked by the MFMA's op_sel)
  v8i a[MTW][KC][4];
  uint32_t sa[MTW][KC];
  auto load_a = [&](int64_t c) {
    const int cr = lane >> 2, cp = lane & 3;
    const int from = 4 * (4 * r + q);
#pragma unroll
    for (int mi = 0; mi < MTW; ++mi) {
      const int64_t r0 = 16 * (MTW * wv + mi) + cr;
      const int64_t row = r0 < p.M ? r0 : p.M - 1;  // rows past M: any valid row
      const uint8_t* arow = p.a + row * p.lda;
      const uint8_t* srow = static_cast<const uint8_t*>(p.sa) + sa_row_offset(p, row);
#pragma unroll
      for (int u = 0; u < KC; ++u) {
        const int64_t kt = c * KC + u;
        uint4 lo[4], hi[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t k0 = kt * kTileK + 128 * j;
          const int64_t kc = k0 < p.K ? k0 : p.K - 128;
          lo[j] = *reinterpret_cast<const uint4*>(arow + kc + 16 * cp);
          hi[j] = *reinterpret_cast<const uint4*>(arow + kc + 64 + 16 * cp);
        }
        const uint32_t sd = *reinterpret_cast<const uint32_t*>(srow + scale_slice_offset(p, kt * kTileK + 128 * cp));
        uint32_t packed = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t x[8] = {lo[j].x, lo[j].y, lo[j].z, lo[j].w, hi[j].x, hi[j].y, hi[j].z, hi[j].w};
          int y[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) y[e] = __builtin_amdgcn_ds_bpermute(from, (int)x[e]);
          const bool in = kt * kTileK + 128 * j < p.K;
          a[mi][u][j] = in ? v8i{y[0], y[1], y[2], y[3], y[4], y[5], y[6], y[7]} : v8i{0, 0, 0, 0, 0, 0, 0, 0};
          const uint32_t sj = ((uint32_t)__builtin_amdgcn_ds_bpermute(4 * (4 * r + j), (int)sd) >> (8 * q)) & 0xFFu;
          packed |= (in ? sj : 0u) << (8 * j);
        }
        sa[mi][u] = packed;
      }
    }
  };

  v4f held[HELD][MTW];
  int64_t held_item[HELD];
  int nheld = 0;

  // prologue: the ring's first R - 1 items, then the first item's activations (the weight
  // stream from HBM starts at once; the activations come from L2 meanwhile)
#pragma unroll
  for (int k = 0; k < R - 1; ++k)
    if (i0 + k < i1)
      chunk_copy_item<FMT, KC, W>(p, ring + k * S::BYTES, (i0 + k) / g.ntiles, (i0 + k) % g.ntiles, wv, lane);
  int64_t cur_chunk = i0 / g.ntiles;
  load_a(cur_chunk);

  for (int64_t i = i0; i < i1; ++i) {
    const int64_t c = i / g.ntiles;
    if (c != cur_chunk) {  // a new chunk: its activation fragments (at most once more per workgroup)
      load_a(c);
      cur_chunk = c;
    }
    const int slot = (int)((i - i0) % R);
    // item i's copies are complete once at most those of the later items in flight remain
    const int later = (int)(i1 - 1 - i < R - 2 ? i1 - 1 - i : R - 2);
    if (scale_wave) chunk_wait<S::C_SCALE, R - 2>(later);
    else chunk_wait<S::C_PLAIN, R - 2>(later);
    asm volatile("s_barrier" ::: "memory");  // every wave's copies of item i have landed
    if (i + R - 1 < i1) {
      // the slot of item i - 1, free: every wave is past its reads (the barrier above)
      chunk_copy_item<FMT, KC, W>(p, ring + ((i + R - 1 - i0) % R) * S::BYTES, (i + R - 1) / g.ntiles,
                                  (i + R - 1) % g.ntiles, wv, lane);
    }
    const uint8_t* sl = ring + slot * S::BYTES;
    v4f acc[MTW];
#pragma unroll
    for (int mi = 0; mi < MTW; ++mi) acc[mi] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < KC; ++u) {
      const uint32_t sb = *reinterpret_cast<const uint32_t*>(sl + S::SB + u * 256 + lane * 4);
      const uint8_t* tile = sl + S::B + u * S::CH * 1024 + lane * 16;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v8i b;
        if (FMT == kE4M3) {
          const uint4 lo = *reinterpret_cast<const uint4*>(tile + 2 * j * 1024);
          const uint4 hi = *reinterpret_cast<const uint4*>(tile + (2 * j + 1) * 1024);
          b = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        } else {  // FP6: slice j's 24 bytes start at byte 0 (even j) or 8 (odd j) of chunk 3j/2
          const uint8_t* base = tile + ((3 * j) >> 1) * 1024;
          const int odd = j & 1;
          const uint2 d0 = *reinterpret_cast<const uint2*>(base + 8 * odd);
          const uint2 d1 = *reinterpret_cast<const uint2*>(base + (odd ? 1024 : 8));
          const uint2 d2 = *reinterpret_cast<const uint2*>(base + (odd ? 1032 : 1024));
          b = v8i{(int)d0.x, (int)d0.y, (int)d1.x, (int)d1.y, (int)d2.x, (int)d2.y, 0, 0};
        }
#pragma unroll
        for (int mi = 0; mi < MTW; ++mi) {
          if (j == 0) acc[mi] = mfma_step_packed<FMT, 0>(a[mi][u][j], b, acc[mi], sa[mi][u], sb);
          if (j == 1) acc[mi] = mfma_step_packed<FMT, 1>(a[mi][u][j], b, acc[mi], sa[mi][u], sb);
          if (j == 2) acc[mi] = mfma_step_packed<FMT, 2>(a[mi][u][j], b, acc[mi], sa[mi][u], sb);
          if (j == 3) acc[mi] = mfma_step_packed<FMT, 3>(a[mi][u][j], b, acc[mi], sa[mi][u], sb);
        }
      }
    }
    // kept in registers and stored in batches after a full wait: a store's completion
    // counts in vmcnt and need not come in order with the copies, so no store may be in
    // flight while the counts above wait for copies
#pragma unroll
    for (int mi = 0; mi < MTW; ++mi) held[nheld][mi] = acc[mi];
    held_item[nheld] = i;
    if (++nheld == HELD || i + 1 == i1) {
      chunk_wait_vm<0>();
#pragma unroll
      for (int h = 0; h < HELD; ++h) {
        if (h >= nheld) break;
        const int64_t hc = held_item[h] / g.ntiles, hn = held_item[h] % g.ntiles;
        // lane (q, r) holds rows 16 m + 4 q + e of m-tile m, column 16 hn + r
        const int64_t col = hn * 16 + r;
        if (col >= p.N) continue;
#pragma unroll
        for (int mi = 0; mi < MTW; ++mi)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int64_t row = 16 * (MTW * wv + mi) + 4 * q + e;
            if (row >= p.M) continue;
            if (g.nchunks > 1) p.partial[(hc * p.M + row) * p.N + col] = held[h][mi][e];
            else p.out[row * p.ldc + col] = out_bits(p, held[h][mi][e], col);
          }
      }
      chunk_wait_vm<0>();
      nheld = 0;
    }
  }
}

namespace {
template <int FMT, int KC, int MTW>
hipError_t launch_chunk_fmt(const GemmParams& p, const ChunkGrid& g, hipStream_t s) {
  const int64_t G = g.items < cu_count() ? g.items : cu_count();
  hipLaunchKernelGGL((gemm_chunk_kernel<FMT, KC, MTW>), dim3((unsigned)G), dim3(64 * (8 / MTW)), 0, s, p, g);
  return hipGetLastError();
}
}  // namespace

bool chunk_gemm_eligible(int64_t M, int64_t K, int fmt) {
  return M >= 1 && M <= 128 && K % 128 == 0 && K >= 128 && (fmt == kE4M3 || fmt == kE2M3 || fmt == kE3M2);
}

int64_t chunk_count(int64_t K, int kc) {  // kc: super-tiles per chunk
  const int64_t KT = (K + kTileK - 1) / kTileK;
  return (KT + kc - 1) / kc;
}

hipError_t launch_gemm_chunk(int fmt, const GemmParams& p, hipStream_t s) {
  ChunkGrid g;
  g.nchunks = chunk_count(p.K, kChunkSuperTiles);
  g.ntiles = (p.N + 15) / 16;
  g.items = g.nchunks * g.ntiles;
  if (fmt == kE4M3) return launch_chunk_fmt<kE4M3, kChunkSuperTiles, 1>(p, g, s);
  if (fmt == kE2M3) return launch_chunk_fmt<kE2M3, kChunkSuperTiles, 1>(p, g, s);
  if (fmt == kE3M2) return launch_chunk_fmt<kE3M2, kChunkSuperTiles, 1>(p, g, s);
  return hipErrorInvalidValue;
}

bool chunk_gemm_preferred(int64_t M, int64_t N, int64_t K) {
  // measured fastest (a per-shape sweep over every kernel, tile and split) only where the
  // whole K is one chunk and there are more n-tiles than CUs, so that a workgroup's
  // activation fragments serve more than one weight tile: W6A8 N = 4608 / 6144, K = 2048
  // at M = 72..128, 11.8-12.2 against 12.7-14.0 us for the wide kernel.  With at most one
  // n-tile per CU the generic or the wide kernel won (N = 512 / 2048, K = 256 / 2048:
  // 5.0-7.5 against 8.1-8.7 us), and with several chunks the partials cost more (c2
  // M = 128: 22.2 against 17.0 us).
  return M >= 64 && M <= 128 && chunk_count(K, kChunkSuperTiles) == 1 && (N + 15) / 16 > cu_count();
}

}  // namespace mxl
