// Weight-streaming GEMM for decode-sized M (M <= 16) on gfx950.
//
// With at most 16 activation rows the GEMM is a stream over the weights: each
// weight byte is used once, so the kernel is bound by HBM bandwidth and the
// design goal is to keep enough weight bytes in flight on every CU.
//
//   * A workgroup of W = ceil(KT / RUN) wavefronts owns one n-tile (16 weight
//     rows) at a time; wave w takes the RUN consecutive 512-wide super-tiles
//     starting at RUN w, so each of its four K128 slices per super-tile has a
//     static position (fixed chunk offsets, fixed op_sel of the E8M0 dwords).
//   * Workgroups are persistent over n-tiles (g, g + G, g + 2G, ... with G at
//     most one per CU).  Each wave keeps its activation fragments and scales in
//     registers for every n-tile (the at most 16 activation rows are the same
//     throughout); the first weights are requested before them.
//   * Weight fragments are loaded straight from the MFMA-tiled layout into
//     registers (1 KiB per wave per load).  With RUN = 1 they are double-
//     buffered by n-tile: the next n-tile's loads are issued before the current
//     MFMAs, in a loop unrolled by two with unconditional loads (the last
//     prefetch re-reads a valid tile), so the compiler's own waits stay exact.
//   * The W per-wave 16 x 16 fp32 partials are summed in LDS in wave order
//     (double-buffered by n-tile, one barrier per n-tile), rounded to bf16,
//     bias added in bf16.
//   * Block-FP8 (E4M3 weights with an fp32 scale per 128 x 128 block, activations
//     with an fp32 scale per row per 128): each K128 slice is one unscaled MFMA
//     folded with fma(raw, sa * sb, acc); the activation scales of a lane's four
//     output rows stay in registers beside its fragments, the weight block scales
//     ride with each n-tile's weights.  At most eight waves (K <= 8192).
#include "gemm_common.h"

#include <map>
#include <mutex>
#include <utility>


namespace mxl {

namespace {

constexpr int kStreamMaxWaves = 16;
// the in-register MXFP8 quantizer for up to 16 rows: at most this many super-tiles (one
// per wave, two waves per SIMD), so the raw rows' registers fit beside the weights
// (K <= 4096; at ten waves the 168-register budget spilled)
constexpr int kStreamQuantRowsMaxKT = 8;
// the slice-by-slice form of it (ROWP = 12 + rule): fewer registers (156), so up to
// twelve waves (K <= 6144, three per SIMD)
constexpr int kStreamQuantRowsSliceMaxKT = 12;
constexpr int64_t kStreamMaxK = 12288;  // two super-tiles per wave, at most twelve waves
// block-FP8 keeps four fp32 activation scales per slice in registers: at most eight
// waves (two per SIMD, 256 registers each), one super-tile each up to K = 4096, two up to 8192
constexpr int kStreamBlockMaxWaves = 8;
constexpr int64_t kStreamBlockMaxK = 8192;
constexpr int kStreamGroupedMaxExperts = 1024;
// one-launch producer + GEMM: a scratch slot holds [16, K] codes then the scales
constexpr int kFusedSlots = 64;
constexpr int64_t kFusedCodeBytes = 16 * kStreamMaxK;
constexpr int64_t kFusedSlotBytes = kFusedCodeBytes + 16 * (kStreamMaxK / 32);
static_assert(kFusedSlotBytes % 256 == 0, "slots stay 256-byte aligned");
static_assert(16 * (kStreamBlockMaxK / 128) * 4 <= 16 * (kStreamMaxK / 32), "block-FP8 scales fit the slot");

// Buffer descriptors over a scratch slot's codes and scales: loads and stores through them
// carry the sc1 policy (coherent at device scope: no L2 writeback or invalidate is needed
// to hand data between workgroups on different XCDs), and offsets past the slot read 0.
typedef unsigned int v4u32 __attribute__((ext_vector_type(4)));
constexpr int kCpolSc1 = 16;  // the sc1 bit of a buffer access's cache-policy operand
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slot_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

template <int FMT>
struct StreamFmt {
  static constexpr int CH = FmtTraits<FMT>::CH;
  static constexpr int DW = FMT == kE4M3 ? 8 : 6;  // operand dwords per lane per K128 slice
};

template <int FMT, int RUN, bool BLOCK = false>
struct StreamB {
  uint32_t d[RUN][4][StreamFmt<FMT>::DW];
  uint32_t s[RUN];  // tiled E8M0 dword of the super-tile (byte j = slice j)
  float sbv[BLOCK ? RUN : 1][4];  // block-FP8: the weight block scale of slice j (fp32 [N/128, K/128])
  uint32_t bias;    // bf16 bias bits of output column (t % 16) of the n-tile, loaded with the
                    // weights and converted at use, so no wait lands between the prefetches
};

// Weight operands of super-tile kt of n-tile nt (the lane's 16 bytes of every chunk);
// with MX scales also the lane's tiled E8M0 dword.
template <int FMT, bool BLOCK = false>
__device__ __forceinline__ void stream_load_tile(const uint8_t* w, const uint8_t* sw, int64_t KT, int64_t nt,
                                                 int64_t kt, int lane, uint32_t (&d)[4][StreamFmt<FMT>::DW],
                                                 uint32_t& sd) {
  constexpr int CH = StreamFmt<FMT>::CH;
  const uint8_t* tile = w + (nt * KT + kt) * (CH * 1024) + lane * 16;
  uint4 c[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) c[i] = *reinterpret_cast<const uint4*>(tile + i * 1024);
  if (FMT == kE4M3) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 lo = c[2 * j], hi = c[2 * j + 1];
      d[j][0] = lo.x; d[j][1] = lo.y; d[j][2] = lo.z; d[j][3] = lo.w;
      d[j][4] = hi.x; d[j][5] = hi.y; d[j][6] = hi.z; d[j][7] = hi.w;
    }
  } else {  // the lane's 24 dwords; slice j takes dwords [6 j, 6 j + 6)
    uint32_t all[24];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      all[4 * i] = c[i].x; all[4 * i + 1] = c[i].y; all[4 * i + 2] = c[i].z; all[4 * i + 3] = c[i].w;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int k = 0; k < 6; ++k) d[j][k] = all[6 * j + k];
  }
  if (BLOCK) sd = 0;
  else sd = *reinterpret_cast<const uint32_t*>(sw + (nt * KT + kt) * 256 + lane * 4);
}

template <int FMT, int RUN, bool BLOCK>
__device__ __forceinline__ void stream_load_b(const GemmParams& p, const uint8_t* w, const uint8_t* sw, int64_t nt,
                                              const int64_t (&kt)[RUN], int lane, StreamB<FMT, RUN, BLOCK>& b) {
#pragma unroll
  for (int u = 0; u < RUN; ++u) stream_load_tile<FMT, BLOCK>(w, sw, p.KT, nt, kt[u], lane, b.d[u], b.s[u]);
  if constexpr (BLOCK) {  // block scales of the n-tile's 128-row block, clamped inside K
    const int64_t G = p.K / 128;
    const float* sbp = reinterpret_cast<const float*>(sw) + (nt / 8) * G;
#pragma unroll
    for (int u = 0; u < RUN; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t gi = kt[u] * 4 + j;
        b.sbv[u][j] = sbp[gi < G ? gi : G - 1];
      }
  }
  const int64_t col = nt * 16 + (lane & 15);
  // unconditional load (without a bias, any valid halfword: the value is unused)
  const uint16_t* bp = p.bias ? p.bias + (col < p.N ? col : p.N - 1) : reinterpret_cast<const uint16_t*>(sw);
  b.bias = *bp;
}

// Block-FP8: each K128 slice is one unscaled MFMA folded in slice order with
// fma(raw, sa * sb, acc) (sa: the fp32 activation scales of the lane's four rows);
// even and odd slices feed two accumulators, summed at the end.
template <int RUN>
__device__ __forceinline__ v4f stream_mfma_block(const v8i (&a)[RUN][4], const float4 (&s4)[RUN][4],
                                                 const StreamB<kE4M3, RUN, true>& b, const bool (&valid)[RUN]) {
  v4f acc[2] = {};
#pragma unroll
  for (int u = 0; u < RUN; ++u) {
    if (!valid[u]) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t* d = b.d[u][j];
      const v8i bf = v8i{(int)d[0], (int)d[1], (int)d[2], (int)d[3], (int)d[4], (int)d[5], (int)d[6], (int)d[7]};
      const v4f raw = mfma_raw<kE4M3>(a[u][j], bf);
      const float sbv = b.sbv[u][j];
      const float f[4] = {s4[u][j].x * sbv, s4[u][j].y * sbv, s4[u][j].z * sbv, s4[u][j].w * sbv};
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[j & 1][i] = __builtin_fmaf(raw[i], f[i], acc[j & 1][i]);
    }
  }
  v4f out;
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = acc[0][i] + acc[1][i];
  return out;
}

// With two super-tiles per wave, two independent accumulators (even and odd
// slices) summed at the end: two short MFMA dependency chains instead of one long
// one.  One super-tile keeps a single chain (its register budget is tighter).
template <int FMT, int RUN>
__device__ __forceinline__ v4f stream_mfma(const v8i (&a)[RUN][4], const uint32_t (&sa)[RUN][4],
                                           const StreamB<FMT, RUN>& b, const bool (&valid)[RUN]) {
  v4f acc[RUN] = {};
#pragma unroll
  for (int u = 0; u < RUN; ++u) {
    if (!valid[u]) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t* d = b.d[u][j];
      const v8i bf = FMT == kE4M3 ? v8i{(int)d[0], (int)d[1], (int)d[2], (int)d[3], (int)d[4], (int)d[5], (int)d[6], (int)d[7]}
                                  : v8i{(int)d[0], (int)d[1], (int)d[2], (int)d[3], (int)d[4], (int)d[5], 0, 0};
      if (j == 0) acc[0] = mfma_step<FMT, 0>(a[u][j], bf, acc[0], sa[u][j], b.s[u]);
      if (j == 1) acc[RUN - 1] = mfma_step<FMT, 1>(a[u][j], bf, acc[RUN - 1], sa[u][j], b.s[u]);
      if (j == 2) acc[0] = mfma_step<FMT, 2>(a[u][j], bf, acc[0], sa[u][j], b.s[u]);
      if (j == 3) acc[RUN - 1] = mfma_step<FMT, 3>(a[u][j], bf, acc[RUN - 1], sa[u][j], b.s[u]);
    }
  }
  v4f out;
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = RUN == 2 ? acc[0][i] + acc[RUN - 1][i] : acc[0][i];
  return out;
}

// stream_mfma<FMT, 1> with the lane's four activation scale bytes packed in one dword
// (byte j: slice j): the same MFMA chain, in a quarter of the scale registers.
template <int FMT>
__device__ __forceinline__ v4f stream_mfma_packed(const v8i (&a)[4], uint32_t sa, const StreamB<FMT, 1>& b) {
  v4f acc = {};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t* d = b.d[0][j];
    const v8i bf = FMT == kE4M3 ? v8i{(int)d[0], (int)d[1], (int)d[2], (int)d[3], (int)d[4], (int)d[5], (int)d[6], (int)d[7]}
                                : v8i{(int)d[0], (int)d[1], (int)d[2], (int)d[3], (int)d[4], (int)d[5], 0, 0};
    if (j == 0) acc = mfma_step_packed<FMT, 0>(a[j], bf, acc, sa, b.s[0]);
    if (j == 1) acc = mfma_step_packed<FMT, 1>(a[j], bf, acc, sa, b.s[0]);
    if (j == 2) acc = mfma_step_packed<FMT, 2>(a[j], bf, acc, sa, b.s[0]);
    if (j == 3) acc = mfma_step_packed<FMT, 3>(a[j], bf, acc, sa, b.s[0]);
  }
  return acc;
}

// Spin bound of the grid handoff below (polls about 128 cycles apart: about a second).
// Every workgroup of a launch is resident at once (at most one per CU), so the bound is
// only reached if that fails; the launch then completes with unspecified outputs.
constexpr uint32_t kHandoffSpinLimit = 1u << 23;

// Producer wave of a weight-streaming GEMM with its activation producer in the same
// launch (FPROD: 1, 2 = SwiGLU -> MXFP8 under that rule; 4 + rule = the MXFP8 activation
// quantizer; 8 = the block-FP8 quantizer).  The producer waves of the G workgroups split
// the [M, K] producer work in the standalone kernels' lane mapping (lane task i: 8
// values, row i / (K/8), elements 8 (i % (K/8)) .. + 7; four lanes per 32-block, sixteen
// per 128-group) and the standalone kernels' arithmetic, so codes and scales are bit-
// identical to theirs; they store them into p.a / p.sa with device-coherent stores, the
// codes (and the MX scales) in MFMA fragment order, the block-FP8 scales column-major
// [K/128, M]; rows M..15 of the fragments are left unwritten (their outputs are not
// stored, and an MFMA output row depends on its own activation row only).  Then
// the grid handoff: each producer wave waits for its stores to complete, counts itself in
// at fsync[0] and waits until all G have; the last to leave resets fsync[0] and fsync[32]
// (the departures) to zero for the next launch on the slot.  A final barrier releases its
// workgroup's weight waves, whose weights were requested at launch and which read the
// codes with device-coherent loads.
template <int FPROD>
__device__ __forceinline__ void stream_produce(const GemmParams& p, int lane, int64_t g, int64_t G) {
  constexpr bool SWI = FPROD < 4, BLK = FPROD == 8;
  constexpr int RULE = FPROD & 3;
  constexpr int U = 2;  // lane tasks per pass, their loads issued together
  const int64_t per_row = p.K >> 3;
  const int64_t tasks = p.M * per_row;  // a multiple of 16: K % 128 == 0
  uint8_t* codes = const_cast<uint8_t*>(p.a);
  const __amdgpu_buffer_rsrc_t srs_ = slot_rsrc(p.sa, kFusedSlotBytes - kFusedCodeBytes);
  for (int64_t base = g * 64; base < tasks; base += G * 64 * U) {
    uint4 raw[U][SWI ? 2 : 1];
    int64_t row[U], off[U];
    bool live[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t task = base + (int64_t)u * G * 64 + lane;
      live[u] = task < tasks;  // whole 4- (16-) lane groups: base is a multiple of 64
      const int64_t tc = live[u] ? task : tasks - 1;
      row[u] = tc / per_row;
      off[u] = (tc - row[u] * per_row) * 8;
      const uint16_t* src = p.fsrc + row[u] * p.fsrc_ld + off[u];
      raw[u][0] = *reinterpret_cast<const uint4*>(src);
      if constexpr (SWI) raw[u][SWI ? 1 : 0] = *reinterpret_cast<const uint4*>(src + p.K);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float v[8];
      uint32_t pk[2];
      if constexpr (BLK) {
        bf16x8_to_f32(raw[u][0], v);
        quiet8(v);
        const float scale = block_fp8_quant8(v, pk);
        if (live[u] && (lane & 15) == 0)
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, scale), srs_,
                                                (int)(((off[u] >> 7) * p.M + row[u]) * 4), 0, kCpolSc1);
      } else {
        uint32_t s;
        if constexpr (SWI) {
          float gt[8], up[8];
          bf16x8_to_f32(raw[u][0], gt);
          bf16x8_to_f32(raw[u][SWI ? 1 : 0], up);
          swiglu8<RULE>(gt, up, v);
          s = quant8x4<RULE, true>(v, pk);
        } else {
          s = quant8x4_bf16<RULE>(raw[u][0], pk);
        }
        if (live[u] && (lane & 3) == 0) {
          // block b of the row: super-tile b / 16, slice (b % 16) / 4, lane group b % 4
          const int64_t b = off[u] >> 5;
          const int64_t at = (b >> 4) * 256 + (16 * (b & 3) + row[u]) * 4 + ((b & 15) >> 2);
          __builtin_amdgcn_raw_buffer_store_b8((uint8_t)s, srs_, (int)at, 0, kCpolSc1);
        }
      }
      if (live[u]) {
        // fragment order: K index k of slice s sits in lane 16 ((k % 64) / 16) + row, byte
        // 16 (k / 64) + k % 16 of the lane's 32
        const int64_t k = off[u] & 127;
        const int64_t at = (off[u] >> 7) * 2048 + (16 * ((k & 63) >> 4) + row[u]) * 32 + 16 * (k >> 6) + (k & 15);
        __hip_atomic_store(reinterpret_cast<uint64_t*>(codes + at), (uint64_t)pk[0] | (uint64_t)pk[1] << 32,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  // Every store above is device-coherent (sc1); once they are complete the workgroup
  // counts itself in.  The codes are read back with device-coherent loads as well, so no
  // L2 writeback or invalidate is involved (measured: a release/acquire fence pair per
  // workgroup multiplied the launch time).
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  uint32_t* arrive = p.fsync;
  uint32_t* depart = p.fsync + 32;
  if (lane == 0) {
    __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t spins = 0;
    while (__hip_atomic_load(arrive, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (uint32_t)G &&
           ++spins < kHandoffSpinLimit)
      __builtin_amdgcn_s_sleep(2);
    if (__hip_atomic_fetch_add(depart, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)G - 1) {
      __hip_atomic_store(arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(depart, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  asm volatile("s_barrier" ::: "memory");
}

}  // namespace

// ROWP >= 0 (one activation row): each wave computes its own super-tiles' MXFP8 codes
// and scales from the bf16 row p.a while its weights are in flight, with the standalone
// producers' arithmetic:
//   ROWP = rule (0..2): p.a is the gate/up row [2K], swiglu8 + quant8x4 under the rule;
//   ROWP = 4 + rule:    p.a is the row [K], quiet8 + quant8x4 under the rule (the
//                       activation quantizer's).
//
// FPROD >= 0 (M <= 16, the activation producer in the same launch): the last wave of
// each workgroup is a producer wave (stream_produce) that writes its share of the
// [M, K] codes and scales into p.a / p.sa and takes part in a grid handoff; the other
// waves request their first weights, wait at a workgroup barrier for that handoff and
// then read the codes (device-coherent loads, sc1) as the two-launch path's GEMM does,
// with the same MFMA chain and sums.
template <int FMT, int RUN, bool DB, bool BLOCK, int ROWP = -1, int FPROD = -1>
__global__ __launch_bounds__(BLOCK ? 512 : (ROWP >= 12 ? 64 * kStreamQuantRowsSliceMaxKT : ROWP >= 8 ? 64 * kStreamQuantRowsMaxKT : (RUN == 1 ? 1024 : 768)))
void gemm_stream_kernel(GemmParams p) {
  static_assert(!BLOCK || FMT == kE4M3, "block-FP8 weights are E4M3");
  static_assert(ROWP < 0 || BLOCK == (ROWP == 16), "ROWP 16 is the block-FP8 row, the others feed MX GEMMs");
  static_assert(ROWP < 0 || FPROD < 0, "one producer scheme per launch");
  static_assert(FPROD < 0 || (FPROD == 8) == BLOCK, "block-FP8 GEMMs take the block-FP8 quantizer");
  static_assert(ROWP < 8 || ROWP == 16 || RUN == 1, "the in-register quantizer takes one super-tile per wave");
  constexpr bool ROW = ROWP >= 0 && ROWP < 8, SWI = ROWP >= 0 && ROWP < 4;
  constexpr bool QROWS = ROWP >= 8 && ROWP < 16, QSLICE = ROWP >= 12 && ROWP < 16;
  constexpr bool BROW = ROWP == 16;  // one bf16 row, block-FP8 quantized by every wavefront
  constexpr bool FUSED = FPROD >= 0;
  constexpr int RRULE = ROWP & 3;
  __shared__ float red[2][kStreamMaxWaves][4][64];
  const int t = threadIdx.x, lane = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int W = (int)(blockDim.x >> 6) - (FUSED ? 1 : 0);  // weight waves
  const int r = lane & 15, q = lane >> 4;
  const int64_t ntiles = (p.N + 15) / 16;
  const int64_t G = gridDim.x, g = blockIdx.x;
  if constexpr (FUSED) {
    if (wv == W) {
      stream_produce<FPROD>(p, lane, g, G);
      return;
    }
  }
  const uint8_t* w = p.w;
  const uint8_t* sw = static_cast<const uint8_t*>(p.sw);

  // this wave's super-tiles; waves past the end re-read the last tile and add nothing
  int64_t kt[RUN];
  bool valid[RUN];
#pragma unroll
  for (int u = 0; u < RUN; ++u) {
    const int64_t k = (int64_t)wv * RUN + u;
    valid[u] = k < p.KT;
    kt[u] = valid[u] ? k : p.KT - 1;
  }

  // Weights first (the HBM stream is the critical path), then this wave's activation
  // fragments and scales, kept in registers for every n-tile (rows >= M read row
  // M - 1 and are never stored; loads are clamped inside K so all are unconditional)
  const int64_t count = g < ntiles ? (ntiles - g + G - 1) / G : 0;  // n-tiles of this workgroup
  // The fused row's bf16 pieces (gate and up for SwiGLU) are requested before the weights:
  // vector loads complete in issue order, so the producer arithmetic then waits for these
  // loads only and runs while the weights stream in.
  uint4 gu_raw[ROW || BROW ? RUN : 1][SWI ? 2 : 1];
  if constexpr (ROW || BROW) {
    const uint16_t* gu = reinterpret_cast<const uint16_t*>(p.a);
#pragma unroll
    for (int u = 0; u < RUN; ++u) {
      const int64_t k0 = kt[u] * kTileK + (lane >> 2) * 32 + (lane & 3) * 8;
      const int64_t kc = k0 < p.K ? k0 : p.K - 8;  // blocks past K: any valid data, zeroed below
      gu_raw[u][0] = *reinterpret_cast<const uint4*>(gu + kc);
      if constexpr (SWI) gu_raw[u][SWI ? 1 : 0] = *reinterpret_cast<const uint4*>(gu + p.K + kc);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep them ahead of the weight loads
  }
  // QROWS: fragment lane (q, r)'s bf16 pieces of row r (rows past M read row M - 1 and are
  // never stored), K values 16 q .. 16 q + 15 and 64 + 16 q .. + 15 of each slice, also
  // requested ahead of the weights
  uint4 qr_raw[QROWS ? 4 : 1][QROWS ? 4 : 1];
  if constexpr (QROWS) {
    const uint16_t* xrow = reinterpret_cast<const uint16_t*>(p.a) + (r < p.M ? r : p.M - 1) * p.lda;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t k0 = kt[0] * kTileK + 128 * j;
      const int64_t kc = k0 < p.K ? k0 : p.K - 128;  // slices past K: any valid data, zeroed below
      const uint16_t* b0 = xrow + kc + 16 * q;
      qr_raw[j][0] = *reinterpret_cast<const uint4*>(b0);
      qr_raw[j][1] = *reinterpret_cast<const uint4*>(b0 + 8);
      qr_raw[j][2] = *reinterpret_cast<const uint4*>(b0 + 64);
      qr_raw[j][3] = *reinterpret_cast<const uint4*>(b0 + 72);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep them ahead of the weight loads
  }
  if constexpr (FUSED) {
    // the producer wave has seen every workgroup's codes complete: this barrier hands
    // them over.  The weights are requested only after it: requested at launch they fill
    // the memory queues, and every round trip of the handoff (the producer's inputs, its
    // stores, the counter) then waits behind them -- measured 6-11 us per launch more than
    // the producer and the GEMM as two launches.
    asm volatile("s_barrier" ::: "memory");
  }
  StreamB<FMT, RUN, BLOCK> b0;
  stream_load_b<FMT, RUN, BLOCK>(p, w, sw, g < ntiles ? g : ntiles - 1, kt, lane, b0);
  // the activation side: plain loads, or device-coherent ones from the scratch slot
  const __amdgpu_buffer_rsrc_t a_rs = slot_rsrc(p.a, FUSED ? kFusedCodeBytes : 0);
  const __amdgpu_buffer_rsrc_t s_rs = slot_rsrc(p.sa, FUSED ? kFusedSlotBytes - kFusedCodeBytes : 0);
  auto load_a16 = [&](const uint8_t* ptr) -> uint4 {
    if constexpr (FUSED) {
      const v4u32 v = __builtin_amdgcn_raw_buffer_load_b128(a_rs, (int)(ptr - p.a), 0, kCpolSc1);
      return make_uint4(v.x, v.y, v.z, v.w);
    } else {
      return *reinterpret_cast<const uint4*>(ptr);
    }
  };
  auto load_s32 = [&](const void* ptr) -> uint32_t {
    if constexpr (FUSED)
      return __builtin_amdgcn_raw_buffer_load_b32(
          s_rs, (int)(static_cast<const uint8_t*>(ptr) - static_cast<const uint8_t*>(p.sa)), 0, kCpolSc1);
    else
      return *static_cast<const uint32_t*>(ptr);
  };
  // The loads are row-major -- lane l reads piece l % 4 of row l / 4, so four
  // neighbouring lanes move one row's 64 bytes in one access (lanes on sixteen
  // rows, the fragment order, would cost an access each) -- and a lane-permute
  // hands fragment lane 16 q + r its piece q of row r.
  v8i a[RUN][4];
  uint32_t sraw[RUN][4];
  float4 s4[BLOCK ? RUN : 1][4];  // block-FP8: fp32 scales of the lane's output rows 4 q .. 4 q + 3, slice j
  if constexpr (BLOCK && !BROW) {
    const float* sa = static_cast<const float*>(p.sa);  // column-major [K/128, M]
    const int64_t G = p.K / 128;
    int64_t rows[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rows[i] = 4 * q + i < p.M ? 4 * q + i : p.M - 1;
    // the lane's four rows are consecutive floats of the group's column: one 16-byte
    // load where they all lie inside M and the column keeps 16-byte alignment
    bool vec4 = false;
    if constexpr (!FUSED) vec4 = p.M % 4 == 0 && (reinterpret_cast<uintptr_t>(sa) & 15) == 0 && 4 * q + 3 < p.M;
#pragma unroll
    for (int u = 0; u < RUN; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t gi = kt[u] * 4 + j < G ? kt[u] * 4 + j : G - 1;
        if (vec4)
          s4[u][j] = *reinterpret_cast<const float4*>(sa + gi * p.M + 4 * q);
        else
          s4[u][j] = float4{__builtin_bit_cast(float, load_s32(sa + gi * p.M + rows[0])),
                            __builtin_bit_cast(float, load_s32(sa + gi * p.M + rows[1])),
                            __builtin_bit_cast(float, load_s32(sa + gi * p.M + rows[2])),
                            __builtin_bit_cast(float, load_s32(sa + gi * p.M + rows[3]))};
      }
  }
  if constexpr (ROW) {
    // lanes 4 b .. 4 b + 3 own 32-block b of the super-tile (8 values each, the producer's
    // lane mapping).  Fragment lane 16 q + r of slice j holds K values 16 q .. 16 q + 15
    // (dwords 0-3) and 64 + 16 q .. 64 + 16 q + 15 (dwords 4-7) of the slice, the layout the
    // unfused path loads: dword 4 h + d is word d % 2 of lane 4 b + 2 (q % 2) + d / 2 with
    // b = 4 j + 2 h + q / 2.  Its scale is block 4 j + q's code, placed in byte q where the
    // scale dword of the unfused path has it.
#pragma unroll
    for (int u = 0; u < RUN; ++u) {
      float v[8];
      uint32_t pk[2], sc;
      if constexpr (SWI) {
        float g[8], up[8];
        bf16x8_to_f32(gu_raw[u][0], g);
        bf16x8_to_f32(gu_raw[u][SWI ? 1 : 0], up);
        swiglu8<RRULE>(g, up, v);
        sc = quant8x4<RRULE, true>(v, pk);
      } else {
        sc = quant8x4_bf16<RRULE>(gu_raw[u][0], pk);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int b = 4 * j + 2 * (e >> 2) + (q >> 1);
          y[e] = __builtin_amdgcn_ds_bpermute(4 * (4 * b + 2 * (q & 1) + ((e & 3) >> 1)), (int)pk[e & 1]);
        }
        a[u][j] = v8i{y[0], y[1], y[2], y[3], y[4], y[5], y[6], y[7]};
        sraw[u][j] = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * 4 * (4 * j + q), (int)sc) << (8 * q);
      }
    }
  } else if constexpr (QROWS) {
    // The MXFP8 quantizer of up to 16 rows in the fragment registers (the standalone
    // kernel's arithmetic): lane (q, r)'s two 16-value pieces of slice j are halves of
    // blocks q / 2 and 2 + q / 2 of the slice, whose other halves lane q ^ 1 (lane xor 16,
    // the same row) holds, so one row swap completes each block amax; the MFMA takes lane
    // (q, r)'s scale for block q, which lane q = 3 (block 1) or q = 0 (block 2) computed,
    // or the lane itself (blocks 0 and 3).  Both exchanges are VALU lane swaps
    // (v_permlane16_swap / v_permlane32_swap), not LDS round trips: with one wave per
    // SIMD nothing else hides their latency.
    auto piece = [&](int j, int h, uint32_t* d) {
      d[0] = qr_raw[j][2 * h].x;     d[1] = qr_raw[j][2 * h].y;     d[2] = qr_raw[j][2 * h].z;
      d[3] = qr_raw[j][2 * h].w;     d[4] = qr_raw[j][2 * h + 1].x; d[5] = qr_raw[j][2 * h + 1].y;
      d[6] = qr_raw[j][2 * h + 1].z; d[7] = qr_raw[j][2 * h + 1].w;
    };
    auto place = [&](int j, const uint32_t (*c)[4], const uint32_t* sc) {
      a[0][j] = v8i{(int)c[0][0], (int)c[0][1], (int)c[0][2], (int)c[0][3],
                    (int)c[1][0], (int)c[1][1], (int)c[1][2], (int)c[1][3]};
      // x = rows (sc0.0, sc0.1, sc1.0, sc1.1), y = rows (sc0.2, sc0.3, sc1.2, sc1.3): even
      // q takes x (its own block 0, or lane q = 0's block 2), odd q takes y (lane q = 3's
      // block 1, or its own block 3)
      const auto xy = __builtin_amdgcn_permlane32_swap(sc[0], sc[1], false, false);
      sraw[0][j] = ((q & 1) ? xy[1] : xy[0]) << (8 * q);
    };
    if constexpr (QSLICE) {
      // Slice by slice (an empty asm chains each slice's raw values to the previous
      // slice's scale, so the compiler does not hoist every slice's work: 156 registers),
      // one wave-uniform branch per slice; otherwise as below.
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (j > 0) {
#pragma unroll
          for (int h = 0; h < 4; ++h)
            asm volatile("" : "+v"(qr_raw[j][h].x), "+v"(qr_raw[j][h].y), "+v"(qr_raw[j][h].z), "+v"(qr_raw[j][h].w)
                         : "v"(sraw[0][j > 0 ? j - 1 : 0]));
        }
        uint32_t c[2][4], sc[2];
        bool fast[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          uint32_t d[8];
          piece(j, h, d);
          uint32_t mb = amax_bf16_bits<8, false>(d);
          const auto mm = __builtin_amdgcn_permlane16_swap(mb, mb, false, false);
          mb = mm[0] > mm[1] ? mm[0] : mm[1];
          sc[h] = 255u;
          if constexpr (RRULE == kFloorCarry175) sc[h] = scale_floor_carry175(mb);
          if constexpr (RRULE == kCeilDiv448) sc[h] = pow2_ceil_div448(u2f(mb << 16)) >> 23;
          fast[h] = RRULE != kRpUe8m0 && mb <= 0x7F80u && sc[h] < 255u;
        }
        if (__builtin_amdgcn_ballot_w64(!(fast[0] && fast[1])) == 0) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            uint32_t d[8];
            piece(j, h, d);
            codes_bf16_scaled<4, false>(d, sc[h], c[h]);
          }
        } else {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            float m = 0.0f;
            float v[16];
            if (!fast[h]) {
              bf16x8_to_f32(qr_raw[j][2 * h], v);
              bf16x8_to_f32(qr_raw[j][2 * h + 1], v + 8);
              quiet8(v);
              quiet8(v + 8);
#pragma unroll
              for (int i = 0; i < 16; ++i) m = __builtin_fmaxf(m, __builtin_fabsf(v[i]));
            }
            // (outside the branch, whose condition the two lanes of a block share)
            const auto ms = __builtin_amdgcn_permlane16_swap(f2u(m), f2u(m), false, false);
            if (fast[h]) {
              uint32_t d[8];
              piece(j, h, d);
              codes_bf16_scaled<4, false>(d, sc[h], c[h]);
            } else {
              sc[h] = quant_block_codes<RRULE, false, 16>(v, __builtin_fmaxf(u2f(ms[0]), u2f(ms[1])), c[h]);
            }
          }
        }
        place(j, c, sc);
      }
    } else {
      // Every block amax as bf16 magnitude bits, NaNs included (above 0x7F80 when one is
      // present); rows {0, 1} and {2, 3} side by side, so the max is the xor-16 max.  With
      // power-of-two scales, no NaN in the wave's blocks and no E8M0 code 255 (rule 0 wraps
      // there for amax below 2^-119, rule 1 at an infinite amax) the scaled conversion codes
      // straight from bf16, one branch for the wave; otherwise each block whose scale or
      // values need it takes the standalone quantizer's binary32 arithmetic.
      uint32_t sfs[4][2];
      bool fast = RRULE != kRpUe8m0;
  #pragma unroll
      for (int j = 0; j < 4; ++j)
  #pragma unroll
        for (int h = 0; h < 2; ++h) {
          uint32_t d[8];
          piece(j, h, d);
          uint32_t mb = amax_bf16_bits<8, false>(d);
          const auto mm = __builtin_amdgcn_permlane16_swap(mb, mb, false, false);
          mb = mm[0] > mm[1] ? mm[0] : mm[1];
          uint32_t sf = 255u;
          if constexpr (RRULE == kFloorCarry175) sf = scale_floor_carry175(mb);
          if constexpr (RRULE == kCeilDiv448) sf = pow2_ceil_div448(u2f(mb << 16)) >> 23;
          sfs[j][h] = sf;
          fast = fast && mb <= 0x7F80u && sf < 255u;
        }
      if (__builtin_amdgcn_ballot_w64(!fast) == 0) {
  #pragma unroll
        for (int j = 0; j < 4; ++j) {
          uint32_t c[2][4];
  #pragma unroll
          for (int h = 0; h < 2; ++h) {
            uint32_t d[8];
            piece(j, h, d);
            codes_bf16_scaled<4, false>(d, sfs[j][h], c[h]);
          }
          place(j, c, sfs[j]);
        }
      } else {
  #pragma unroll
        for (int j = 0; j < 4; ++j) {
          // slice j's raw values "depend" on slice j - 1's result (an empty asm), so the
          // compiler converts one slice at a time instead of hoisting every slice's floats
          if (j > 0) {
  #pragma unroll
            for (int h = 0; h < 4; ++h)
              asm volatile("" : "+v"(qr_raw[j][h].x), "+v"(qr_raw[j][h].y), "+v"(qr_raw[j][h].z), "+v"(qr_raw[j][h].w)
                           : "v"(sraw[0][j > 0 ? j - 1 : 0]));
          }
          uint32_t c[2][4], sc[2];
  #pragma unroll
          for (int h = 0; h < 2; ++h) {
            uint32_t d[8];
            piece(j, h, d);
            const uint32_t mb = amax_bf16_bits<8, false>(d);
            const auto mm = __builtin_amdgcn_permlane16_swap(mb, mb, false, false);
            const bool blk_fast = RRULE != kRpUe8m0 && (mm[0] > mm[1] ? mm[0] : mm[1]) <= 0x7F80u && sfs[j][h] < 255u;
            float m = 0.0f;
            float v[16];
            if (!blk_fast) {
              bf16x8_to_f32(qr_raw[j][2 * h], v);
              bf16x8_to_f32(qr_raw[j][2 * h + 1], v + 8);
              quiet8(v);
              quiet8(v + 8);
  #pragma unroll
              for (int i = 0; i < 16; ++i) m = __builtin_fmaxf(m, __builtin_fabsf(v[i]));
            }
            // (outside the branch, whose condition the two lanes of a block share)
            const auto ms = __builtin_amdgcn_permlane16_swap(f2u(m), f2u(m), false, false);
            if (blk_fast) {
              codes_bf16_scaled<4, false>(d, sfs[j][h], c[h]);
              sc[h] = sfs[j][h];
            } else {
              sc[h] = quant_block_codes<RRULE, false, 16>(v, __builtin_fmaxf(u2f(ms[0]), u2f(ms[1])), c[h]);
            }
          }
          place(j, c, sc);
        }
      }
    }
  } else if constexpr (BROW) {
    // The block-FP8 quantizer of the row (the standalone kernel's quiet8 +
    // block_fp8_quant8: lanes 16 j .. 16 j + 15 hold slice j's 128 values, 8 each, the
    // group's amax by xor-shuffles over them), every wavefront its own super-tiles.  The
    // codes reach the fragment lanes as in the MX row above (lane l holds values 8 l ..
    // 8 l + 7 of the super-tile); every output row of the lane is row 0 (M = 1), so its
    // four activation scales are the slice's.  A slice past K (a part super-tile) takes
    // the last slice's scale, as the two-launch path's clamped scale load does; its
    // weights are zero.
#pragma unroll
    for (int u = 0; u < RUN; ++u) {
      float v[8];
      uint32_t pk[2];
      bf16x8_to_f32(gu_raw[u][0], v);
      quiet8(v);
      const float scale = block_fp8_quant8(v, pk);
      const int64_t last = (p.K / 128 - 1) - kt[u] * 4;  // the super-tile's last slice inside K
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int b = 4 * j + 2 * (e >> 2) + (q >> 1);
          y[e] = __builtin_amdgcn_ds_bpermute(4 * (4 * b + 2 * (q & 1) + ((e & 3) >> 1)), (int)pk[e & 1]);
        }
        a[u][j] = v8i{y[0], y[1], y[2], y[3], y[4], y[5], y[6], y[7]};
        const int js = j <= last ? j : (int)last;
        const float sj = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * 16 * js, __builtin_bit_cast(int, scale)));
        s4[u][j] = float4{sj, sj, sj, sj};
      }
    }
  } else if constexpr (FUSED) {
    // the scratch holds the codes in fragment order (stream_produce): slice s's 32 bytes
    // of fragment lane l at 2048 s + 32 l, so each lane loads its own fragments; the MX
    // scale dword of lane l for super-tile kt at 256 kt + 4 l holds slice j's code in byte
    // j, placed in byte q where the two-launch path's scale dword has it
    const int64_t nsl = p.K >> 7;
#pragma unroll
    for (int u = 0; u < RUN; ++u) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t sl = kt[u] * 4 + j < nsl ? kt[u] * 4 + j : nsl - 1;  // clamped inside K
        const uint4 lo = load_a16(p.a + sl * 2048 + lane * 32);
        const uint4 hi = load_a16(p.a + sl * 2048 + lane * 32 + 16);
        a[u][j] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      }
      if constexpr (!BLOCK) {
        const uint32_t sd = load_s32(static_cast<const uint8_t*>(p.sa) + kt[u] * 256 + lane * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) sraw[u][j] = ((sd >> (8 * j)) & 0xFFu) << (8 * q);
      }
    }
  } else {
    const int cr = lane >> 2, cp = lane & 3;
    const int64_t row = cr < p.M ? cr : p.M - 1;
    // (block-FP8 has no E8M0 scales: any valid address, the dword is unused)
    // rows < 16: in the swizzled layout row r's dword of slice 0 sits at 16 r (one 128-row tile)
    const int64_t srs = p.sa_swz ? 16 : p.K / 32;
    const uint8_t* srow = BLOCK ? p.a : static_cast<const uint8_t*>(p.sa) + row * srs;
    const uint8_t* arow = p.a + row * p.lda;
    const int from = 4 * (4 * r + q);  // byte address of the source lane (4 r + q)
#pragma unroll
    for (int u = 0; u < RUN; ++u) {
      uint4 lo[4], hi[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t k0 = kt[u] * kTileK + 128 * j;
        const int64_t kc = k0 < p.K ? k0 : p.K - 128;
        lo[j] = load_a16(arow + kc + 16 * cp);
        hi[j] = load_a16(arow + kc + 64 + 16 * cp);
      }
      // scale dword of slice cp (E8M0 of blocks 4 cp .. 4 cp + 3 of the super-tile)
      const int64_t ks = kt[u] * kTileK + 128 * cp;
      const uint32_t sd = BLOCK ? 0u : load_s32(srow + scale_slice_offset(p, ks));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t x[8] = {lo[j].x, lo[j].y, lo[j].z, lo[j].w, hi[j].x, hi[j].y, hi[j].z, hi[j].w};
        int y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = __builtin_amdgcn_ds_bpermute(from, (int)x[e]);
        a[u][j] = v8i{y[0], y[1], y[2], y[3], y[4], y[5], y[6], y[7]};
        sraw[u][j] = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (4 * r + j), (int)sd);
      }
    }
  }
  // slices past the end of K (the upper half of a K % 512 == 256 tail) contribute zero
  uint32_t sa[RUN][4];
#pragma unroll
  for (int u = 0; u < RUN; ++u)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool in = kt[u] * kTileK + 128 * j < p.K;
      sa[u][j] = in ? (sraw[u][j] >> (8 * q)) & 0xFFu : 0u;
      if (!in) a[u][j] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
    }

  // reduce the W wave partials of n-tile nt (buffer `buf`) and store the output elements
  auto finish = [&](const v4f& acc, uint32_t bias_bits, int64_t nt, int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) red[buf][wv][i][lane] = acc[i];
    // LDS handover without a memory fence (a fence would also drain the weight
    // prefetch in flight): wait for this wave's LDS writes, then the barrier
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    for (int e = t; e < 256; e += 64 * W) {  // fewer than four waves loop
      const int i = e >> 6, l = e & 63;
      float sum = red[buf][0][i][l];
      for (int v = 1; v < W; ++v) sum += red[buf][v][i][l];
      const int64_t row = 4 * (l >> 4) + i, col = nt * 16 + (l & 15);
      if (row < p.M && col < p.N)
        p.out[row * p.ldc + col] = out_bits(sum, p.alpha, p.out_f16, p.bias != nullptr, (uint16_t)bias_bits);
    }
  };

  auto mma = [&](const StreamB<FMT, RUN, BLOCK>& b) -> v4f {
    if constexpr (BLOCK) return stream_mfma_block<RUN>(a, s4, b, valid);
    else return stream_mfma<FMT, RUN>(a, sa, b, valid);
  };
  if (DB) {
    StreamB<FMT, RUN, BLOCK> b1;
    for (int64_t j = 0; j < count; j += 2) {
      const int64_t nt0 = g + j * G;
      // prefetch the second n-tile of the pair (or re-read the first)
      const int64_t nt1 = j + 1 < count ? nt0 + G : nt0;
      stream_load_b<FMT, RUN, BLOCK>(p, w, sw, nt1, kt, lane, b1);
      finish(mma(b0), b0.bias, nt0, 0);
      const int64_t nt2 = j + 2 < count ? nt0 + 2 * G : nt1;
      stream_load_b<FMT, RUN, BLOCK>(p, w, sw, nt2, kt, lane, b0);
      if (j + 1 < count) finish(mma(b1), b1.bias, nt1, 1);
    }
  } else {
    for (int64_t j = 0; j < count; ++j) {
      const int64_t nt = g + j * G;
      if (j > 0) stream_load_b<FMT, RUN, BLOCK>(p, w, sw, nt, kt, lane, b0);
      finish(mma(b0), b0.bias, nt, (int)(j & 1));
    }
  }
}

// rounds of weight fragments in each wave's register ring in the grouped variant
constexpr int kStreamGroupedDepth = 4;

// Grouped (MoE) weight-streaming GEMM.  A persistent workgroup owns one unit -- up to
// 16 MT routed rows (MT m-tiles) of one expert -- at a time and streams all of that
// expert's weight n-tiles past the unit's activation fragments, which each wave
// gathers once into registers.  Its WK x NW waves split K (wave w takes super-tile
// w % WK) and N (n-lane w / WK takes n-tiles w / WK, + NW, ...), so a CU keeps many
// weight fragments in flight even when K is one super-tile; per round of NW n-tiles
// the WK partials of each are summed in LDS in K order (one super-tile: stored
// directly).  Units are numbered expert by expert (a block scan of the experts' unit
// counts in LDS), so the launch needs no host-side counts.  Every m-tile's product is
// the same MFMA chain whatever MT is, so the MT variants give identical bits.
// Waves per workgroup: MT = 1 (a few rows per expert): eight, each keeping
// kStreamGroupedDepth - 1 rounds of weight fragments in flight in a register ring (a
// round's tiles arrive one HBM latency after their request, so with one round ahead a
// round costs a whole latency under load).  MT > 1: four, whose activation fragments
// (32 MT registers per super-tile) need the registers of a whole SIMD.
template <int FMT, int MT>
constexpr int stream_grouped_waves() { return MT > 1 ? 4 : 8; }

// Activation producers fused into the grouped kernel (prod != 0): the workgroup
// computes its unit's MXFP8 operands -- codes [ROWS][K] then E8M0 [ROWS][K/32], rows
// past the unit repeating its last row -- into LDS with the standalone producers'
// arithmetic and lane mapping (four lanes per 32-element block), so the codes are
// those quant_mxfp8_kernel / swiglu_mxfp8_kernel would write:
//   prod 1: MXFP8 quantization of the gathered bf16 rows A[row_index[r] / row_div]
//           (row stride lda), rule `rule`;
//   prod 2: SwiGLU of the unit's bf16 gate/up rows (gate columns [0, K), up [K, 2K),
//           row stride lda) then MXFP8, rule `rule`.
// One producer item is the 8 values lane c % 4 of 32-block (c / 4) % (K / 32) of unit row
// (c / 4) / (K / 32) owns.  Its loads are split from its arithmetic so that the kernel can
// issue the first item's loads ahead of the unit's first weight loads: vector loads
// complete in issue order, so the arithmetic then waits for these loads only, not for the
// weights behind them.
struct ProduceIn {
  uint4 x, y;  // prod 1: the 8 bf16 values (x); prod 2: gate (x) and up (y)
};

__device__ __forceinline__ void produce_load(const GemmParams& p, int prod, int64_t lo, int64_t hi, int c,
                                             ProduceIn& in) {
  const int bpr = (int)(p.K / 32);
  const int sub = c & 3, blk = (c >> 2) % bpr, rloc = (c >> 2) / bpr;
  int64_t row = lo + rloc;
  if (row >= hi) row = hi - 1;
  const uint16_t* src = reinterpret_cast<const uint16_t*>(p.a);
  if (prod == 1) {
    const int64_t arow = p.row_index ? (int64_t)(p.row_index[row] / p.row_div) : row;
    in.x = *reinterpret_cast<const uint4*>(src + arow * p.lda + blk * 32 + sub * 8);
  } else {
    const uint16_t* gp = src + row * p.lda + blk * 32 + sub * 8;
    in.x = *reinterpret_cast<const uint4*>(gp);
    in.y = *reinterpret_cast<const uint4*>(gp + p.K);
  }
}

template <int ROWS, int PRODUCER, int RULE>
__device__ __forceinline__ void produce_store(const GemmParams& p, int c, bool live, const ProduceIn& in,
                                              uint8_t* stage) {
  const int64_t K = p.K;
  const int bpr = (int)(K / 32);
  const int sub = c & 3, blk = (c >> 2) % bpr, rloc = (c >> 2) / bpr;
  float v[8];
  uint32_t packed[2], sc;
  if constexpr (PRODUCER == 1) {
    sc = quant8x4_bf16<RULE>(in.x, packed);
  } else {
    float g[8], u[8];
    bf16x8_to_f32(in.x, g);
    bf16x8_to_f32(in.y, u);
    // two halves, so that the scheduler does not interleave all eight exp sequences: a
    // spill reload here would wait (vmcnt) for the unit's first weights as well
    swiglu8<RULE, 4>(g, u, v);
    __builtin_amdgcn_sched_barrier(0);
    swiglu8<RULE, 4>(g + 4, u + 4, v + 4);
    sc = quant8x4<RULE, true>(v, packed);
  }
  if (live) {
    *reinterpret_cast<uint2*>(stage + rloc * K + blk * 32 + sub * 8) = make_uint2(packed[0], packed[1]);
    if (sub == 0) stage[ROWS * K + rloc * bpr + blk] = (uint8_t)sc;
  }
}

// Activation producers fused into the grouped kernel (prod != 0): the workgroup
// computes its unit's MXFP8 operands -- codes [ROWS][K] then E8M0 [ROWS][K/32], rows
// past the unit repeating its last row -- into LDS with the standalone producers'
// arithmetic and lane mapping (four lanes per 32-element block), so the codes are
// those quant_mxfp8_kernel / swiglu_mxfp8_kernel would write:
//   producer 1: MXFP8 quantization of the gathered bf16 rows A[row_index[r] / row_div]
//               (row stride lda), scale rule RULE;
//   producer 2: SwiGLU of the unit's bf16 gate/up rows (gate columns [0, K), up [K, 2K),
//               row stride lda) then MXFP8, rule RULE.
// (Each producer and rule is its own instantiation: one kernel holding all three rules'
// code would hold every rule's registers.)
// Only the unit's rows are produced (the gather reads its padding rows from the last
// one): items = rows x K/32 x 4.  Items and thread counts are multiples of four, so the
// four lanes of a block are live together; threads past the end redo the last block
// without storing.  With EARLY, `first` holds item t's loads, issued by the caller.
template <int ROWS, int PRODUCER, int RULE, bool EARLY>
__device__ __forceinline__ void grouped_produce(const GemmParams& p, int64_t lo, int64_t hi, uint8_t* stage, int t,
                                                int nthreads, ProduceIn first) {
  const int items = (int)(hi - lo) * (int)(p.K / 32) * 4;
  if constexpr (!EARLY) produce_load(p, PRODUCER, lo, hi, t < items ? t : items - 4 + (t & 3), first);
  produce_store<ROWS, PRODUCER, RULE>(p, t < items ? t : items - 4 + (t & 3), t < items, first, stage);
  for (int base = nthreads; base < items; base += nthreads) {
    const int c = base + t < items ? base + t : items - 4 + (t & 3);
    ProduceIn in;
    produce_load(p, PRODUCER, lo, hi, c, in);
    produce_store<ROWS, PRODUCER, RULE>(p, c, base + t < items, in, stage);
  }
}

// Device-coherent access to the routed output of a combine-fused launch (COMB): buffer
// loads and stores with the sc1 cache policy, the bits the compiler gives agent-scope
// atomic loads and stores, so a row stored by a workgroup on one XCD and read by one on
// another needs no L2 write-back or invalidation (device-scope fences around every unit
// cost 141.7 -> 225.2 us at c5 T = 128, 233 -> 650 us at T = 2048).  Byte offsets are
// 32-bit: the host bounds the routed output below 2 GiB.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t routed_rsrc(const GemmParams& p) {
  return __builtin_amdgcn_make_buffer_rsrc(p.out, (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ void store16_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off, uint4 v) {
  typedef int v4i_ __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(v4i_{(int)v.x, (int)v.y, (int)v.z, (int)v.w}, r, off, 0, kCpolSc1);
}
__device__ __forceinline__ uint4 load16_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCpolSc1);
  return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}

// Most routes per token of a combine-fused launch (the route table of each token a
// unit completes is kept in LDS).
constexpr int kCombineMaxTopk = 16;

// Weighted combine of the ntok tokens a unit completed (COMB): out[tok] = bf16(sum over k
// ascending of w[tok, k] * y[pos[tok, k]]) in fp32 (the moe_reduce_kernel arithmetic).
// Items (token, eight columns) are spread over every thread of the workgroup, and an
// item's row loads are all issued before its sums, so each thread has up to topk
// loads in flight.
__device__ __forceinline__ void grouped_combine(const GemmParams& p, int ntok, const int32_t* tok,
                                                const int32_t (*pos)[kCombineMaxTopk],
                                                const float (*wt)[kCombineMaxTopk], int t, int nthreads) {
  const __amdgpu_buffer_rsrc_t ry = routed_rsrc(p);
  const int topk = p.comb_topk;
  const int per = (int)(p.N / 8);
  for (int it = t; it < ntok * per; it += nthreads) {
    const int i = it / per, c = it - i * per;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
    for (int k0 = 0; k0 < topk; k0 += 8) {
      uint4 raw[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int32_t q = k0 + u < topk ? pos[i][k0 + u] : -1;
        raw[u] = q >= 0 ? load16_coherent(ry, (uint32_t)(((int64_t)q * p.ldc + 8 * c) * 2)) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (k0 + u >= topk || pos[i][k0 + u] < 0) continue;
        const float wk = wt[i][k0 + u];
        float v[8];
        bf16x8_to_f32(raw[u], v);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float term = v[e] * wk;
          acc[e] = acc[e] + term;
        }
      }
    }
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = (uint32_t)f32_to_bf16(acc[2 * e]) | ((uint32_t)f32_to_bf16(acc[2 * e + 1]) << 16);
    *reinterpret_cast<uint4*>(p.comb_out + (int64_t)tok[i] * p.N + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// COMB: the weighted combine runs inside the kernel.  A unit stores its routed rows
// device-coherently (sc1), waits for those stores to complete, and each row adds one to
// its token's counter (a device-scope atomic); the unit whose row completes a token's
// count (its routes with inv >= 0) reads the token's rows device-coherently, writes the
// combined row and resets the counter to zero for the next launch.  Tokens with no routed
// row are written as zeros at the start.  Every token's last row is stored by some unit,
// so every combined row is written once, by whichever unit finishes it; no wave waits on
// another.  K must be one super-tile per wave (WK = 1: the whole-line store path).  Used
// with the 16-row units (the small-batch schedule): at c5 T = 128 the layer took 141.0 us
// with the combine as its own launch; at T = 2048 (96-row units, ~96 tokens completed per
// unit, 64 MB of routed rows re-read at the units' ends) the in-kernel combine measured
// 573 against 231 us and is not used.
template <int FMT, int MT, int PROD, bool COMB = false>
__global__ __launch_bounds__((64 * stream_grouped_waves<FMT, MT>())) void gemm_stream_grouped_kernel(GemmParams p, int E,
                                                                                                int WK, int NW) {
  // PROD = 4 producer + rule: producer 0 (none), 1 (quantization) or 2 (SwiGLU), rule the
  // MXFP8 scale rule of the produced operands
  constexpr int prod = PROD >> 2, RULE = PROD & 3;
  constexpr int WAVES = stream_grouped_waves<FMT, MT>();
  // prod != 0: the unit's produced operands (grouped_produce), sized at launch
  extern __shared__ __attribute__((aligned(16))) uint8_t stage_act[];
  constexpr int ROWS = 16 * MT;
  __shared__ float red[2][WAVES][MT][4][64];
  // one super-tile: the round's NW adjacent n-tiles of all waves side by side in bf16, so
  // that each row's 16 NW columns (whole 128-byte lines) are stored together
  // (double-buffered by round; row stride 16 NW + 8 halfwords keeps 16-byte pieces
  // aligned).  Per-wave 32-byte row pieces left the lines to be merged in L2 between the
  // weight reads: 68.9 -> 64.9 us at c5 T = 2048 (96-row units), 47.1 -> 46.5 at T = 128.
  __shared__ __attribute__((aligned(16))) uint16_t wstage[2][ROWS][16 * WAVES + 8];
  int wbuf = 0;
  __shared__ int32_t sh_pre[kStreamGroupedMaxExperts + 1];  // units before expert e
  __shared__ int32_t sh_off[kStreamGroupedMaxExperts + 1];  // expert_offsets
  __shared__ int32_t sh_scan[64 * WAVES];
  const int t = threadIdx.x, lane = t & 63, nthreads = (int)blockDim.x;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int kw = wv % WK, nl = wv / WK;
  const int64_t ntiles = (p.N + 15) / 16;

  for (int e = t; e <= E; e += nthreads) sh_off[e] = (int32_t)p.expert_offsets[e];
  __syncthreads();
  // unit counts per thread chunk of experts, then a block-wide inclusive scan
  const int chunk = (E + nthreads - 1) / nthreads;
  const int e0 = t * chunk < E ? t * chunk : E, e1 = e0 + chunk < E ? e0 + chunk : E;
  int cnt = 0;
  for (int e = e0; e < e1; ++e) cnt += (sh_off[e + 1] - sh_off[e] + ROWS - 1) / ROWS;
  sh_scan[t] = cnt;
  __syncthreads();
  for (int off = 1; off < nthreads; off <<= 1) {
    const int v = t >= off ? sh_scan[t - off] : 0;
    __syncthreads();
    sh_scan[t] += v;
    __syncthreads();
  }
  int base = sh_scan[t] - cnt;
  for (int e = e0; e < e1; ++e) {
    sh_pre[e] = base;
    base += (sh_off[e + 1] - sh_off[e] + ROWS - 1) / ROWS;
  }
  if (t == nthreads - 1) sh_pre[E] = sh_scan[t];
  __syncthreads();
  const int units = __builtin_amdgcn_readfirstlane(sh_pre[E]);
  // COMB: the tokens this unit completes, with their routes' rows and weights
  __shared__ int32_t sh_tok[COMB ? ROWS : 1];
  __shared__ int32_t sh_pos[COMB ? ROWS : 1][kCombineMaxTopk];
  __shared__ float sh_wt[COMB ? ROWS : 1][kCombineMaxTopk];
  __shared__ int32_t sh_ntok;
  if constexpr (COMB) {
    // tokens without a routed row (every route dropped) get a zero row
    const int topk = p.comb_topk;
    for (int64_t tk = (int64_t)blockIdx.x * nthreads + t; tk < p.comb_T; tk += (int64_t)gridDim.x * nthreads) {
      bool any = false;
      for (int k = 0; k < topk; ++k) any = any || p.comb_inv[tk * topk + k] >= 0;
      if (!any)
        for (int64_t c = 0; c < p.N / 8; ++c)
          *reinterpret_cast<uint4*>(p.comb_out + tk * p.N + 8 * c) = make_uint4(0u, 0u, 0u, 0u);
    }
  }

  int buf = 0;
  for (int u = (int)blockIdx.x; u < units; u += (int)gridDim.x) {
    // the expert owning unit u: the largest e with sh_pre[e] <= u
    int lo_e = 0, hi_e = E - 1;
    while (lo_e < hi_e) {
      const int mid = (lo_e + hi_e + 1) >> 1;
      if (__builtin_amdgcn_readfirstlane(sh_pre[mid]) <= u) lo_e = mid;
      else hi_e = mid - 1;
    }
    const int e = lo_e;
    const int64_t lo = __builtin_amdgcn_readfirstlane(sh_off[e] + (u - sh_pre[e]) * ROWS);
    const int64_t end = __builtin_amdgcn_readfirstlane(sh_off[e + 1]);
    const int64_t hi = lo + ROWS < end ? lo + ROWS : end;
    const uint8_t* w = p.w + e * p.w_expert_stride;
    const uint8_t* sw = static_cast<const uint8_t*>(p.sw) + e * p.sw_expert_stride;
    const int64_t kt1[1] = {kw < p.KT ? kw : p.KT - 1};
    const bool valid[1] = {kw < p.KT};
    // COMB: the token of this thread's unit row, requested now so that the count at the
    // unit's end does not wait for it
    int64_t ctok = 0;
    if constexpr (COMB) {
      if (t < hi - lo) ctok = p.comb_routes[lo + t] / p.comb_topk;
    }

    // the first round's weights first, then the unit's gathered activation fragments
    StreamB<FMT, 1> b0;
    // 96-row units take their rounds in a rotated order (unit u starts at round
    // u (rounds / 8 + 1) mod rounds), so the CUs do not read the same offsets of their
    // experts' weights at the same time: 73.5 -> 68.6 us at c5 T = 2048 (the 16-row units,
    // measured the same way, lost 1-2 %)
    const int64_t rounds_u = (ntiles + NW - 1) / NW;
    const int64_t rot = MT > 1 ? (int64_t)(u % rounds_u) * (rounds_u / 8 + 1) % rounds_u : 0;
    auto rnd = [&](int64_t round) -> int64_t {
      const int64_t x = round + rot;
      return x < rounds_u ? x : x - rounds_u;
    };
    auto nt_of = [&](int64_t round) -> int64_t {
      const int64_t nt = nl + rnd(round) * NW;
      return nt < ntiles ? nt : ntiles - 1;
    };
    // the SwiGLU producer's first loads go out ahead of the weights (see ProduceIn); the
    // quantizing producer's rows are gathered through row_index, a dependent load, so its
    // loads follow the weights
    ProduceIn first{};
    if constexpr (prod == 2) {
      const int items = (int)(hi - lo) * (int)(p.K / 32) * 4;
      produce_load(p, prod, lo, hi, t < items ? t : items - 4 + (t & 3), first);
      __builtin_amdgcn_sched_barrier(0);  // keep them ahead of the weight loads
    }
    stream_load_b<FMT, 1, false>(p, w, sw, nt_of(0), kt1, lane, b0);
    if constexpr (prod != 0) {
      // every wave has read the previous unit's operands (the s_barrier below the gather
      // orders that); produce this unit's into LDS, then hand them over
      grouped_produce<ROWS, prod, RULE, prod == 2>(p, lo, hi, stage_act, t, nthreads, first);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    v8i a[MT][1][4];
    uint32_t sa[MT > 1 ? 1 : MT][1][4];  // MT = 1: one byte per slice
    uint32_t spk[MT];                    // MT > 1: the four bytes packed (byte j: slice j)
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int cr = lane >> 2, cp = lane & 3;
      int64_t row = lo + 16 * i + cr;
      if (row >= hi) row = hi - 1;  // padding rows read a valid row and are not stored
      const int64_t arow = p.row_index ? (int64_t)(p.row_index[row] / p.row_div) : row;
      const uint8_t* srow = prod ? stage_act + ROWS * p.K + (row - lo) * (p.K / 32)
                                 : static_cast<const uint8_t*>(p.sa) + sa_row_offset(p, arow);
      const uint8_t* ap = prod ? stage_act + (row - lo) * p.K : p.a + arow * p.lda;
      const int from = 4 * (4 * r + q);
      uint4 lo4[4], hi4[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t k0 = kt1[0] * kTileK + 128 * j;
        const int64_t kc = k0 < p.K ? k0 : p.K - 128;
        lo4[j] = *reinterpret_cast<const uint4*>(ap + kc + 16 * cp);
        hi4[j] = *reinterpret_cast<const uint4*>(ap + kc + 64 + 16 * cp);
      }
      const int64_t ks = kt1[0] * kTileK + 128 * cp;
      const uint32_t sd = *reinterpret_cast<const uint32_t*>(
          srow + (prod ? (uint32_t)((ks < p.K ? ks : p.K - 128) >> 7) * 4u : scale_slice_offset(p, ks)));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t x[8] = {lo4[j].x, lo4[j].y, lo4[j].z, lo4[j].w, hi4[j].x, hi4[j].y, hi4[j].z, hi4[j].w};
        int y[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) y[k] = __builtin_amdgcn_ds_bpermute(from, (int)x[k]);
        a[i][0][j] = v8i{y[0], y[1], y[2], y[3], y[4], y[5], y[6], y[7]};
        const uint32_t sraw = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (4 * r + j), (int)sd);
        const bool in = kt1[0] * kTileK + 128 * j < p.K;
        const uint32_t sbyte = in ? (sraw >> (8 * q)) & 0xFFu : 0u;
        if constexpr (MT > 1) spk[i] = (j == 0 ? 0u : spk[i]) | (sbyte << (8 * j));
        else sa[0][0][j] = sbyte;
        if (!in) a[i][0][j] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
    if constexpr (prod != 0) asm volatile("s_waitcnt lgkmcnt(0) vmcnt(0)\n\ts_barrier" ::: "memory");

    // the m-tiles' products of one n-tile (m-tiles without rows are skipped)
    auto mma = [&](const StreamB<FMT, 1>& b, v4f (&acc)[MT]) {
      if constexpr (MT == 1) {
        acc[0] = stream_mfma<FMT, 1>(a[0], sa[0], b, valid);
      } else {
        // every m-tile unconditionally (padding rows are never stored), so the MT
        // independent MFMA chains interleave; a wave past K adds zero
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          acc[i] = stream_mfma_packed<FMT>(a[i][0], spk[i], b);
          if (!valid[0]) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
        }
      }
    };
    // store the round's NW n-tiles: with one super-tile per wave the waves' products meet
    // in LDS and are stored as whole row lines; else the WK partials of each n-tile are
    // summed in LDS in K order
    auto finish = [&](const v4f (&acc)[MT], int64_t round) {
      if (WK == 1) {
        const int64_t nt = nl + rnd(round) * NW;  // NW == WAVES: every wave has its own n-tile
        if (p.N % 8 == 0 && p.ldc % 8 == 0 && ((uintptr_t)p.out & 15) == 0) {
          // every wave puts its 16 MT x 16 tile beside the others' (lane (q, r) holds column
          // r of rows 16 i + 4 q + x), then the workgroup stores 16-byte pieces of each row
          if (nt < ntiles) {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
              for (int x = 0; x < 4; ++x) wstage[wbuf][16 * i + 4 * q + x][16 * nl + r] = f32_to_bf16(acc[i][x]);
          }
          asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
          constexpr int SEG = 2 * WAVES;  // 16-byte pieces per row
          const int64_t col0 = rnd(round) * NW * 16;
          const int nrows = (int)(hi - lo);
          for (int k = 0; k < (ROWS * SEG + 64 * WAVES - 1) / (64 * WAVES); ++k) {
            const int piece = t + 64 * WAVES * k, row = piece / SEG, seg = piece % SEG;
            const int64_t col = col0 + 8 * seg;
            if (row < nrows && col < p.N) {
              const uint4 v = *reinterpret_cast<const uint4*>(&wstage[wbuf][row][8 * seg]);
              if constexpr (COMB)
                store16_coherent(routed_rsrc(p), (uint32_t)(((lo + row) * p.ldc + col) * 2), v);
              else
                *reinterpret_cast<uint4*>(p.out + (lo + row) * p.ldc + col) = v;
            }
          }
          wbuf ^= 1;
          return;
        }
        if (nt >= ntiles) return;
        const int64_t col = nt * 16 + r;
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            const int64_t row = lo + 16 * i + 4 * q + x;
            if (row < hi && col < p.N) p.out[row * p.ldc + col] = f32_to_bf16(acc[i][x]);
          }
        return;
      }
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int x = 0; x < 4; ++x) red[buf][wv][i][x][lane] = acc[i][x];
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      for (int o = t; o < 256 * MT * NW; o += nthreads) {
        const int n = o / (256 * MT), i = (o >> 8) % MT, x = (o >> 6) & 3, l = o & 63;
        float sum;
        if constexpr (MT > 1) {  // at most four K waves: independent reads, summed in K order
          float part[WAVES];
#pragma unroll
          for (int v = 0; v < WAVES; ++v) part[v] = v < WK ? red[buf][n * WK + v][i][x][l] : 0.0f;
          sum = part[0];
#pragma unroll
          for (int v = 1; v < WAVES; ++v)
            if (v < WK) sum += part[v];
        } else {
          sum = red[buf][n * WK][i][x][l];
          for (int v = 1; v < WK; ++v) sum += red[buf][n * WK + v][i][x][l];
        }
        const int64_t nt = n + rnd(round) * NW;
        const int64_t row = lo + 16 * i + 4 * (l >> 4) + x, col = nt * 16 + (l & 15);
        if (nt < ntiles && row < hi && col < p.N) p.out[row * p.ldc + col] = f32_to_bf16(sum);
      }
      buf ^= 1;
    };

    const int64_t rounds = (ntiles + NW - 1) / NW;
    v4f acc[MT];
    {
      // a register ring of kStreamGroupedDepth rounds of weights: round rd + D - 1 requested
      // before round rd is used (past the end: the last round is re-read, and nothing is
      // stored for it)
      constexpr int D = kStreamGroupedDepth;
      StreamB<FMT, 1> ring[D];
      ring[0] = b0;
#pragma unroll
      for (int k = 1; k < D - 1; ++k)
        stream_load_b<FMT, 1, false>(p, w, sw, nt_of(k < rounds ? k : rounds - 1), kt1, lane, ring[k]);
      for (int64_t rd = 0; rd < rounds; rd += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
          const int64_t ahead = rd + k + D - 1;
          stream_load_b<FMT, 1, false>(p, w, sw, nt_of(ahead < rounds ? ahead : rounds - 1), kt1, lane,
                                       ring[(k + D - 1) % D]);
          if (rd + k < rounds) {
            mma(ring[k], acc);
            finish(acc, rd + k);
          }
        }
      }
    }
    if constexpr (COMB) {
      // this unit's rows are stored (coherently) before they are counted
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      if (t == 0) sh_ntok = 0;
      __syncthreads();
      const int nrows = (int)(hi - lo), topk = p.comb_topk;
      if (t < nrows) {
        const int64_t tok = ctok;
        int32_t pos[kCombineMaxTopk];
        int expect = 0;
#pragma unroll
        for (int k = 0; k < kCombineMaxTopk; ++k) {
          pos[k] = k < topk ? p.comb_inv[tok * topk + k] : -1;
          expect += pos[k] >= 0 ? 1 : 0;
        }
        const int old = __hip_atomic_fetch_add(p.comb_cnt + tok, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old + 1 == expect) {
          const int slot = atomicAdd(&sh_ntok, 1);
          sh_tok[slot] = (int32_t)tok;
#pragma unroll
          for (int k = 0; k < kCombineMaxTopk; ++k) {
            sh_pos[slot][k] = pos[k];
            sh_wt[slot][k] = k < topk ? p.comb_w[tok * topk + k] : 0.0f;
          }
          // every route of the token is counted: zero for the next launch (a device-scope store)
          __hip_atomic_store(p.comb_cnt + tok, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      __syncthreads();
      const int ntok = sh_ntok;
      if (ntok > 0) grouped_combine(p, ntok, sh_tok, sh_pos, sh_wt, t, nthreads);
      __syncthreads();  // sh_tok / sh_ntok are reused by the next unit
    }
  }
}

// ------------------------------------------------------------ configuration

// The host side.  gemm_stream_swiglu.hip compiles this file again with
// MXL_STREAM_SWIGLU_ONLY for the one-row SwiGLU launch alone (its own scheduling
// flags); this translation unit holds everything else.
#ifndef MXL_STREAM_SWIGLU_ONLY
// MX: one super-tile per wave (double-buffered) up to 16 super-tiles (K <= 8192);
// two per wave, single-buffered, up to 24 (K <= 12288, twelve waves of at most
// 168 registers).  A super-tile costs 32 + 4 VGPRs of activations and 32 (24
// for FP6) + 1 of weights per buffer.
bool stream_gemm_eligible(int64_t M, int64_t K, bool block) {
  return M >= 1 && M <= 16 && K % 128 == 0 && K >= 128 && K <= (block ? kStreamBlockMaxK : kStreamMaxK);
}

// Compute units of the current device (cached per device).
int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

namespace {
template <int FMT, bool BLOCK>
hipError_t launch_stream_fmt(const GemmParams& p, dim3 grid, hipStream_t s) {
  if (p.KT <= (BLOCK ? kStreamBlockMaxWaves : kStreamMaxWaves)) {
    hipLaunchKernelGGL((gemm_stream_kernel<FMT, 1, true, BLOCK>), grid, dim3((unsigned)(p.KT * 64)), 0, s, p);
  } else {
    hipLaunchKernelGGL((gemm_stream_kernel<FMT, 2, false, BLOCK>), grid, dim3((unsigned)((p.KT + 1) / 2 * 64)), 0,
                       s, p);
  }
  return hipGetLastError();
}
}  // namespace

#endif  // MXL_STREAM_SWIGLU_ONLY

namespace {
// ROWP: the row producer of gemm_stream_kernel (rule of the SwiGLU row, or 4 + rule of
// the quantized row)
template <int FMT, int ROWP>
hipError_t launch_row_fmt(const GemmParams& p, dim3 grid, hipStream_t s) {
  if constexpr (ROWP >= 8) {  // the in-register quantizer: one super-tile per wave
    if (p.KT > (ROWP >= 12 ? kStreamQuantRowsSliceMaxKT : kStreamQuantRowsMaxKT) || p.M > 16)
      return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemm_stream_kernel<FMT, 1, true, false, ROWP>), grid, dim3((unsigned)(p.KT * 64)), 0, s, p);
  } else if (p.KT <= kStreamMaxWaves) {
    hipLaunchKernelGGL((gemm_stream_kernel<FMT, 1, true, false, ROWP>), grid, dim3((unsigned)(p.KT * 64)), 0, s, p);
  } else {
    hipLaunchKernelGGL((gemm_stream_kernel<FMT, 2, false, false, ROWP>), grid,
                       dim3((unsigned)((p.KT + 1) / 2 * 64)), 0, s, p);
  }
  return hipGetLastError();
}
template <int ROWP>
hipError_t launch_row(int fmt, const GemmParams& p, dim3 grid, hipStream_t s) {
  if (fmt == kE4M3) return launch_row_fmt<kE4M3, ROWP>(p, grid, s);
  if (fmt == kE2M3) return launch_row_fmt<kE2M3, ROWP>(p, grid, s);
  if (fmt == kE3M2) return launch_row_fmt<kE3M2, ROWP>(p, grid, s);
  return hipErrorInvalidValue;
}
dim3 row_grid(const GemmParams& p) {
  const int64_t ntiles = (p.N + 15) / 16;
  return dim3((unsigned)(ntiles < cu_count() ? ntiles : cu_count()));
}
}  // namespace

#ifdef MXL_STREAM_SWIGLU_ONLY
bool stream_swiglu_eligible(int64_t M, int64_t K, int rule) {
  return M == 1 && stream_gemm_eligible(1, K, false) && (rule == kCeilDiv448 || rule == kRpUe8m0);
}

hipError_t launch_gemm_stream_swiglu(int fmt, int rule, const GemmParams& p, hipStream_t s) {
  if (rule == kCeilDiv448) return launch_row<kCeilDiv448>(fmt, p, row_grid(p), s);
  if (rule == kRpUe8m0) return launch_row<kRpUe8m0>(fmt, p, row_grid(p), s);
  return hipErrorInvalidValue;
}

#else

bool stream_quant_row_eligible(int64_t M, int64_t K, int rule) {
  return M == 1 && stream_gemm_eligible(1, K, false) && rule >= kFloorCarry175 && rule <= kRpUe8m0;
}

hipError_t launch_gemm_stream_quant_row(int fmt, int rule, const GemmParams& p, hipStream_t s) {
  if (rule == kFloorCarry175) return launch_row<4 + kFloorCarry175>(fmt, p, row_grid(p), s);
  if (rule == kCeilDiv448) return launch_row<4 + kCeilDiv448>(fmt, p, row_grid(p), s);
  if (rule == kRpUe8m0) return launch_row<4 + kRpUe8m0>(fmt, p, row_grid(p), s);
  return hipErrorInvalidValue;
}

bool stream_block_row_eligible(int64_t M, int64_t K) { return M == 1 && stream_gemm_eligible(1, K, true); }

hipError_t launch_gemm_stream_block_row(const GemmParams& p, hipStream_t s) {
  // ROWP 16: the block-FP8 row quantized by every wavefront (E4M3 weights); the waves
  // and super-tiles of the two-launch path's block-FP8 GEMM
  if (p.M != 1) return hipErrorInvalidValue;
  const dim3 grid = row_grid(p);
  if (p.KT <= kStreamBlockMaxWaves)
    hipLaunchKernelGGL((gemm_stream_kernel<kE4M3, 1, true, true, 16>), grid, dim3((unsigned)(p.KT * 64)), 0, s, p);
  else
    hipLaunchKernelGGL((gemm_stream_kernel<kE4M3, 2, false, true, 16>), grid, dim3((unsigned)((p.KT + 1) / 2 * 64)), 0,
                       s, p);
  return hipGetLastError();
}

bool stream_quant_rows_eligible(int64_t M, int64_t K, int rule) {
  return M >= 1 && M <= 16 && stream_gemm_eligible(M, K, false) &&
         (K + kTileK - 1) / kTileK <= kStreamQuantRowsSliceMaxKT && rule >= kFloorCarry175 && rule <= kRpUe8m0;
}

hipError_t launch_gemm_stream_quant_rows(int fmt, int rule, const GemmParams& p, hipStream_t s) {
  // the wave-wide branch up to eight waves (measured faster at c1), the slice-by-slice
  // form past them
  if (p.KT <= kStreamQuantRowsMaxKT) {
    if (rule == kFloorCarry175) return launch_row<8 + kFloorCarry175>(fmt, p, row_grid(p), s);
    if (rule == kCeilDiv448) return launch_row<8 + kCeilDiv448>(fmt, p, row_grid(p), s);
    if (rule == kRpUe8m0) return launch_row<8 + kRpUe8m0>(fmt, p, row_grid(p), s);
  } else {
    if (rule == kFloorCarry175) return launch_row<12 + kFloorCarry175>(fmt, p, row_grid(p), s);
    if (rule == kCeilDiv448) return launch_row<12 + kCeilDiv448>(fmt, p, row_grid(p), s);
    if (rule == kRpUe8m0) return launch_row<12 + kRpUe8m0>(fmt, p, row_grid(p), s);
  }
  return hipErrorInvalidValue;
}

namespace {
template <int MT>
int grouped_waves(int fmt) {
  return fmt == kE4M3 ? stream_grouped_waves<kE4M3, MT>() : stream_grouped_waves<kE2M3, MT>();
}
// LDS bytes of a unit's produced operands (codes + E8M0), 16-byte rounded
int64_t grouped_stage_bytes(int mt, int64_t K) { return ((16 * mt * K * 33 / 32) + 15) / 16 * 16; }

template <int MT>
hipError_t launch_grouped_mt(int fmt, const GemmParams& p, int64_t num_experts, int prod, int rule, hipStream_t s,
                             bool combine) {
  const int waves = grouped_waves<MT>(fmt);
  const int WK = (int)p.KT;
  if (WK < 1 || WK > waves) return hipErrorInvalidValue;
  const int NW = waves / WK;
  // a bound on the units (16 MT routed rows each): every expert adds at most one partial unit
  const int64_t bound = (p.M + 16 * MT - 1) / (16 * MT) + num_experts;
  const int64_t G = bound < cu_count() ? bound : cu_count();
  const dim3 grid((unsigned)G), blk((unsigned)(64 * WK * NW));
  const int E = (int)num_experts;
  const size_t shmem = prod ? (size_t)grouped_stage_bytes(MT, p.K) : 0;
  // the fused producers and the combine are instantiated for the 16-row units only (the
  // schedule that uses them)
  if ((prod || combine) && MT != 1) return hipErrorInvalidValue;
  if (combine && (p.comb_topk < 1 || p.comb_topk > kCombineMaxTopk)) return hipErrorInvalidValue;
#define MXL_GROUPED_LAUNCH(F_, P_, C_)                                                                         \
  hipLaunchKernelGGL((gemm_stream_grouped_kernel<F_, MT, (MT == 1 ? P_ : 0), (MT == 1 && C_)>), grid, blk, shmem, \
                     s, p, E, WK, NW)
  if (prod && (rule < kFloorCarry175 || rule > kRpUe8m0)) return hipErrorInvalidValue;
  const int code = (prod ? 4 * prod + rule : 0) + (combine ? 16 : 0);
  // the combine runs in the down projection: plain operands, or the SwiGLU producer
  // under the two rules the MoE's intermediate activations use
#define MXL_GROUPED_PROD(F_)                            \
  switch (code) {                                       \
    case 0: MXL_GROUPED_LAUNCH(F_, 0, false); break;    \
    case 4: MXL_GROUPED_LAUNCH(F_, 4, false); break;    \
    case 5: MXL_GROUPED_LAUNCH(F_, 5, false); break;    \
    case 6: MXL_GROUPED_LAUNCH(F_, 6, false); break;    \
    case 8: MXL_GROUPED_LAUNCH(F_, 8, false); break;    \
    case 9: MXL_GROUPED_LAUNCH(F_, 9, false); break;    \
    case 10: MXL_GROUPED_LAUNCH(F_, 10, false); break;  \
    case 16: MXL_GROUPED_LAUNCH(F_, 0, true); break;    \
    case 25: MXL_GROUPED_LAUNCH(F_, 9, true); break;    \
    case 26: MXL_GROUPED_LAUNCH(F_, 10, true); break;   \
    default: return hipErrorInvalidValue;               \
  }
  if (fmt == kE4M3) {
    MXL_GROUPED_PROD(kE4M3)
  } else if (fmt == kE2M3) {
    MXL_GROUPED_PROD(kE2M3)
  } else if (fmt == kE3M2) {
    MXL_GROUPED_PROD(kE3M2)
  } else {
    return hipErrorInvalidValue;
  }
#undef MXL_GROUPED_PROD
#undef MXL_GROUPED_LAUNCH
  return hipGetLastError();
}
}  // namespace

bool stream_grouped_eligible(int64_t K, int64_t num_experts, int fmt, int mt) {
  const int waves = mt == 1 ? grouped_waves<1>(fmt) : grouped_waves<kGroupedStreamWideMT>(fmt);
  return (mt == 1 || mt == kGroupedStreamWideMT) && K % 128 == 0 && K >= 128 &&
         (K + kTileK - 1) / kTileK <= waves && num_experts >= 1 && num_experts <= kStreamGroupedMaxExperts;
}

bool stream_grouped_fused_eligible(int64_t K, int64_t num_experts, int fmt, int mt) {
  return stream_grouped_eligible(K, num_experts, fmt, mt) && grouped_stage_bytes(mt, K) <= kGroupedStageMaxBytes;
}

hipError_t launch_gemm_stream_grouped(int fmt, const GemmParams& p, int64_t num_experts, int mt, hipStream_t s,
                                      int prod, int rule, bool combine) {
  if (prod && grouped_stage_bytes(mt, p.K) > kGroupedStageMaxBytes) return hipErrorInvalidValue;
  if (mt == 1) return launch_grouped_mt<1>(fmt, p, num_experts, prod, rule, s, combine);
  if (mt == kGroupedStreamWideMT)
    return launch_grouped_mt<kGroupedStreamWideMT>(fmt, p, num_experts, prod, rule, s, combine);
  return hipErrorInvalidValue;
}

int stream_max_waves(bool block) { return block ? kStreamBlockMaxWaves : kStreamMaxWaves; }

// ------------------------------------------- producer + GEMM in one launch (M <= 16)

// Scratch of the one-launch producer + GEMM: per slot the [16, K] codes (K <= 12288)
// followed by the scales (E8M0 [16, K/32], or block-FP8 fp32 [K/128, 16]), and the grid
// handoff counters, each slot's on its own 256 bytes.  Static device memory: every GPU
// holds its own copy (zero at load) until the process ends; one slot per (device,
// stream), so launches on one stream reuse their slot in order.
__device__ __align__(256) uint8_t g_fused_scratch[kFusedSlots][kFusedSlotBytes];
__device__ __align__(256) uint32_t g_fused_sync[kFusedSlots][64];

// Weight waves of the one-launch variant: RUN = 1 needs KT + 1 waves, RUN = 2
// ceil(KT / 2) + 1, within the kernel's launch bound; the RUN must be the one the
// two-launch GEMM takes for this K (its MFMA chain and wave sums), so KT = 16 (MX) and
// KT = 8 (block-FP8) do not fit.  FP6 weights with RUN = 2 do not fit the registers of
// three waves per SIMD beside the handoff (the compiler spills), so they take two launches.
static int fused_run(int64_t K, bool block, int fmt) {
  const int64_t KT = (K + kTileK - 1) / kTileK;
  const int maxw = block ? kStreamBlockMaxWaves : kStreamMaxWaves;  // RUN = 1 bound, in waves
  const int max2 = block ? kStreamBlockMaxWaves : 12;               // RUN = 2 bound
  if (KT <= maxw) return KT + 1 <= maxw ? 1 : 0;
  return fmt == kE4M3 && (KT + 1) / 2 + 1 <= max2 ? 2 : 0;
}

bool stream_fused_eligible(int64_t M, int64_t K, bool block, int fmt) {
  return stream_gemm_eligible(M, K, block) && fused_run(K, block, fmt) > 0;
}

namespace {
struct FusedSlotTable {
  std::mutex mu;
  std::map<std::pair<int, uintptr_t>, int> slot;
  int used[64] = {};
  uint8_t* scratch[64] = {};
  uint32_t* sync[64] = {};
};
FusedSlotTable& fused_slots() {
  static FusedSlotTable t;
  return t;
}

template <int FMT, bool BLOCK, int FPROD>
hipError_t launch_fused_fmt(const GemmParams& p, dim3 grid, hipStream_t s) {
  if (fused_run(p.K, BLOCK, FMT) == 1)
    hipLaunchKernelGGL((gemm_stream_kernel<FMT, 1, true, BLOCK, -1, FPROD>), grid, dim3((unsigned)((p.KT + 1) * 64)),
                       0, s, p);
  else if constexpr (FMT == kE4M3)
    hipLaunchKernelGGL((gemm_stream_kernel<FMT, 2, false, BLOCK, -1, FPROD>), grid,
                       dim3((unsigned)(((p.KT + 1) / 2 + 1) * 64)), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}
template <int FPROD>
hipError_t launch_fused_prod(int fmt, const GemmParams& p, dim3 grid, hipStream_t s) {
  if (fmt == kE4M3) return launch_fused_fmt<kE4M3, false, FPROD>(p, grid, s);
  if (fmt == kE2M3) return launch_fused_fmt<kE2M3, false, FPROD>(p, grid, s);
  if (fmt == kE3M2) return launch_fused_fmt<kE3M2, false, FPROD>(p, grid, s);
  return hipErrorInvalidValue;
}
}  // namespace

int launch_gemm_stream_fused(int fmt, int prod, GemmParams& p, hipStream_t s, const char* who) {
  const bool block = prod == kFusedBlockFp8;
  if (!stream_fused_eligible(p.M, p.K, block, fmt)) {
    set_error("%s: M=%lld K=%lld does not run as one launch", who, (long long)p.M, (long long)p.K);
    return MXL_EUNSUPPORTED;
  }
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    set_error("%s: no current device", who);
    return MXL_EHIP;
  }
  if (s) {  // the scratch is the current device's: the stream must belong to it
    int sdev = -1;
    if (hipStreamGetDevice(s, &sdev) != hipSuccess || sdev != dev) {
      set_error("%s: the stream's device (%d) is not the current device (%d)", who, sdev, dev);
      return MXL_EINVAL;
    }
  }
  FusedSlotTable& T = fused_slots();
  int slot;
  {
    std::lock_guard<std::mutex> lk(T.mu);
    if (!T.scratch[dev]) {
      void* a = nullptr;
      void* b = nullptr;
      if (hipGetSymbolAddress(&a, HIP_SYMBOL(g_fused_scratch)) != hipSuccess ||
          hipGetSymbolAddress(&b, HIP_SYMBOL(g_fused_sync)) != hipSuccess || !a || !b) {
        set_error("%s: scratch address: %s", who, hipGetErrorString(hipGetLastError()));
        return MXL_EHIP;
      }
      T.scratch[dev] = static_cast<uint8_t*>(a);
      T.sync[dev] = static_cast<uint32_t*>(b);
    }
    const auto key = std::make_pair(dev, (uintptr_t)s);
    auto it = T.slot.find(key);
    if (it == T.slot.end()) {
      if (T.used[dev] >= kFusedSlots) {
        set_error("%s: more than %d streams on device %d use the one-launch producer; use the two calls", who,
                  kFusedSlots, dev);
        return MXL_EUNSUPPORTED;
      }
      it = T.slot.emplace(key, T.used[dev]++).first;
    }
    slot = it->second;
  }
  uint8_t* base = T.scratch[dev] + (int64_t)slot * kFusedSlotBytes;
  p.a = base;
  p.sa = base + kFusedCodeBytes;
  p.fsync = T.sync[dev] + (int64_t)slot * 64;
  p.lda = p.K;
  set_sa_layout(p, 0);
  p.a_rows = p.M;
  const int64_t ntiles = (p.N + 15) / 16;
  const dim3 grid((unsigned)(ntiles < cu_count() ? ntiles : cu_count()));
  hipError_t e = hipErrorInvalidValue;
  switch (prod) {
    case 1: e = launch_fused_prod<1>(fmt, p, grid, s); break;
    case 2: e = launch_fused_prod<2>(fmt, p, grid, s); break;
    case 4: e = launch_fused_prod<4>(fmt, p, grid, s); break;
    case 5: e = launch_fused_prod<5>(fmt, p, grid, s); break;
    case 6: e = launch_fused_prod<6>(fmt, p, grid, s); break;
    case kFusedBlockFp8:
      if (fmt == kE4M3) e = launch_fused_fmt<kE4M3, true, kFusedBlockFp8>(p, grid, s);
      break;
    default: break;
  }
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", who, hipGetErrorString(e));
    return MXL_EHIP;
  }
  return MXL_OK;
}

hipError_t launch_gemm_stream(int fmt, bool block, const GemmParams& p, hipStream_t s) {
  const int64_t ntiles = (p.N + 15) / 16;
  const int64_t G = ntiles < cu_count() ? ntiles : cu_count();
  const dim3 grid((unsigned)G);
  if (block) return fmt == kE4M3 ? launch_stream_fmt<kE4M3, true>(p, grid, s) : hipErrorInvalidValue;
  if (fmt == kE4M3) return launch_stream_fmt<kE4M3, false>(p, grid, s);
  if (fmt == kE2M3) return launch_stream_fmt<kE2M3, false>(p, grid, s);
  if (fmt == kE3M2) return launch_stream_fmt<kE3M2, false>(p, grid, s);
  return hipErrorInvalidValue;
}

#endif  // MXL_STREAM_SWIGLU_ONLY

}  // namespace mxl
