// Wide-tile, LDS-pipelined GEMM for prefill-sized M on gfx950 (MX, block-FP8,
// dense and MoE-grouped).
//
// Workgroup tile: 128 rows x 64*NT columns (NT = 1, 2 or 4), four wavefronts.
// Every wave owns all 8 m-tiles of the 128 rows and its own NT n-tiles; per
// K128 slice it reads each A fragment once from LDS and issues NT MFMAs with it.
//
// All operands reach LDS by direct global->LDS loads (global_load_lds: lane i
// of a wave writes 4 or 16 bytes at LDS base + 4i / 16i, no staging
// registers) into a ring of K128 stage slots (four, or three for NT = 4 whose
// 53 KiB stages would not fit four times), issued two or three stages ahead of
// the MFMAs; the grouped variant runs two workgroups per CU with two slots each,
// one stage ahead.  A slot holds
//   A    8 m-tiles x 2 KiB: chunk (m-tile i, half h) holds rows 16 i + 8 h ..
//        + 7 whole (the slice's 128 bytes per row), the eight 16-byte pieces of
//        row r permuted by piece ^ a_swz(r).  The copy is row-major because the
//        memory pipeline coalesces neighbouring lanes: eight lanes reading one
//        row's 128 bytes move a whole cache line in one request, while lanes on
//        sixteen different rows (MFMA fragment order) cost one access each --
//        measured 10.8 vs 3.0 TB/s for a 16 x 64 B pattern -- and half-line
//        pieces (16 rows x 64 bytes per copy) cost two requests per line: whole
//        rows took 3-7 % off every wide shape.  The permutation keeps the
//        fragment reads (lane 16 q + r: row r, pieces q and 4 + q) free of LDS
//        bank conflicts;
//   B    per wave, its NT n-tiles' 2 KiB of the MFMA-tiled weight (copied
//        verbatim: the tiled layout already is fragment order);
//   SA   the activation scales of the 128 rows (E8M0 dword of blocks 4j..4j+3,
//        or the block-FP8 fp32 scale), copied by waves 0 and 1;
//   SB   per wave, the tiled E8M0 weight-scale dwords of its n-tiles (MX only).
// The copies are issued from inline assembly, so the compiler neither counts
// them nor adds waits of its own: each step waits (vmcnt) for exactly its own
// stage -- the stages issued after it may stay in flight, vector-memory loads
// completing in issue order -- then one barrier hands the slot to all waves and
// frees the slot of the previous step for the next copy.  The slice index of a
// stage is a run-time value, so E8M0 bytes are shifted into place for op_sel 0.
//
// Grid: one workgroup per (m-block, n-block, K split), remapped so that the
// m-blocks sharing a weight slice are consecutive on one XCD (workgroup L runs
// on XCD L % 8) and hit its L2.  K splits (whole 512-wide super-tiles) store their
// fp32 partials straight from the accumulators in MFMA fragment order, one block per
// tile, and a second kernel sums them in split order and writes the rows.  When the whole-K tiles
// leave a partial last round (more tiles than CUs), the same launch runs the
// leftover tiles split in K: workgroup L computes whole-K tile L and then unit L
// of the split leftovers, so no CU waits for a second launch.  The grouped variant
// walks experts' row ranges (expert_offsets) on device, so the launch needs no
// host-side counts.
#include "gemm_common.h"

// the copies set M0 (the LDS base of a global->LDS load) themselves
#pragma clang diagnostic ignored "-Winline-asm"

namespace mxl {

namespace {

template <int MT, int NT, bool BLOCK, int WM = 1>
struct WideSlot {
  static_assert(MT == 4 || MT == 8, "64- or 128-row workgroup tiles");
  static_assert(WM == 1 || (WM == 2 && MT == 8), "two m-groups of waves: 128-row tiles only");
  // MX with NT <= 2: the activation scales live in a separate ring of three
  // super-tile entries (16 MT rows x 16 bytes), filled a super-tile ahead, so a
  // copy moves 16 bytes per row instead of one dword from each row.
  static constexpr bool SA_RING = !BLOCK && NT <= 2;
  static constexpr int A = 0;                               // MT x 2 KiB
  static constexpr int B = MT * 2048;                       // wave w: NT x 2 KiB at B + w NT 2 KiB
  static constexpr int SA = B + 4 * NT * 2048;              // 64 MT bytes, copied by the scale waves (no ring)
  static constexpr int SB = SA + (SA_RING ? 0 : 64 * MT);  // wave w: NT x 256 B (MX)
  static constexpr int BYTES = SB + (BLOCK ? 0 : 4 * NT * 256);
  static constexpr int SLOTS = NT == 4 ? 3 : 4;             // 4 x 53 KiB would not fit the LDS
  static constexpr int SW = MT / 4;                         // scale waves: 0 .. SW - 1, 64 rows each
  static constexpr int RING_ENTRY = 256 * MT;               // scale ring entry: 16 MT rows x 16 bytes
  // WM m-groups of four waves: wave w owns m-tiles (w / 4) MT / WM .. + MT / WM - 1 and the
  // n-tiles of n-group w % 4.  Copies per wave per stage: its share of the A chunks, of its
  // n-group's B chunks (one of the two per n-tile when WM = 2) and of their E8M0 scales (with
  // one n-tile both waves of the group copy it: the same bytes to the same place); the scale
  // waves also copy the activation scales.
  static constexpr int WAVES = 4 * WM;
  static constexpr int ACH = 2 * MT / WAVES;
  static constexpr int BCH = 2 / WM;
  static constexpr int SBC = BLOCK ? 0 : (WM == 1 ? NT : (NT >= 2 ? NT / 2 : 1));
  static constexpr int COPIES = ACH + BCH * NT + SBC;
};

// Ring slots of the grouped variant, which runs two workgroups per CU.
constexpr int kWideGroupedSlots = 2;

typedef __attribute__((address_space(3))) uint8_t lds_u8;

// Piece permutation of row r (0..15) of an m-tile, whose rows are stored whole
// (128 bytes: rows 0..7 in the first 1 KiB chunk, 8..15 in the second): piece p
// of row r sits at 128 (r % 8) + 16 (p ^ a_swz(r)) of its chunk.  For every
// piece p the offsets of rows 0..7 (8..15) are distinct modulo 128 bytes and
// those of rows 0..15 distinct modulo 256 bytes, so a 16-byte fragment read
// meets no bank conflict with either 32 or 64 banks.
__device__ __forceinline__ int a_swz(int r) { return ((r >> 1) ^ ((r & 1) << 2)) & 7; }

__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) { return (uint32_t)(uintptr_t)(const lds_u8*)p; }

// Lane i copies 16 (4) bytes from base + voff to LDS [lds + 16 i] ([lds + 4 i]).
// `base` and `lds` are wave-uniform.
__device__ __forceinline__ void copy16(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(base)
               : "memory", "m0");
}
__device__ __forceinline__ void copy4(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(voff), "s"(base)
               : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt immediate");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without a memory fence (a fence would drain every
// outstanding load): LDS data is handed over by the explicit waits.
__device__ __forceinline__ void wide_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <int MT, int NT, int WM = 1>
struct WideLanes {
  // A chunk c = ACH wv + u (m-tile c / 2, rows 8 (c % 2) .. + 7): copy lane l reads row
  // 8 (c % 2) + l / 8, piece (l % 8) ^ a_swz(row), as row * lda + 16 piece
  uint32_t a_off[2 * MT / (4 * WM)];
  uint32_t sa_off;    // MX: row * K/32; block-FP8: 4 row  (row = t % 16 MT)
  uint32_t sa_piece[4];  // scale ring: lane l of scale wave w reads dword l % 4 of row 4 MT j + 16 w + l / 4
  uint32_t sa_last[4];   // the same for the last super-tile when it is half (K % 512 = 256), from p.sa and
                         // clamped inside the row (its dwords 2, 3 would lie past the row)
  const uint8_t* w_tile[NT];  // wave-uniform: tile (ntile, 0) of each of the wave's n-tiles
  const uint8_t* sw_tile[NT];
};

// Copy K128 stage `t` (super-tile t / 4, slice j = t % 4) into a slot; with
// the scale ring, waves 0 and 1 also copy piece j (32 rows) of the next
// super-tile's activation scales (clamped inside K: a piece past the last
// super-tile is never read).
template <int FMT, int MT, int NT, bool BLOCK, int WM>
__device__ __forceinline__ void wide_copy(const GemmParams& p, uint8_t* slot, int64_t t, int wv, int lane,
                                          const WideLanes<MT, NT, WM>& L, uint8_t* sa_ring) {
  using S = WideSlot<MT, NT, BLOCK, WM>;
  constexpr int CH = FmtTraits<FMT>::CH;
  const int wn = WM == 1 ? wv : wv & 3, wm = WM == 1 ? 0 : wv >> 2;
  const int64_t kt = t >> 2;
  const int j = (int)(t & 3);
#pragma unroll
  for (int u = 0; u < S::ACH; ++u) {  // A chunk ACH wv + u: m-tile c / 2, rows 8 (c % 2) .. + 7, whole rows
    const int c = S::ACH * wv + u;
    copy16(p.a + t * 128, L.a_off[u], lds_addr(slot + S::A + c * 1024));
  }
  // B: the two 1 KiB chunks of the tile that hold slice j (FP6: its 24 bytes per lane
  // straddle two chunks)
  const int c0 = FMT == kE4M3 ? 2 * j : (3 * j) >> 1;
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const uint8_t* tile = L.w_tile[n] + kt * (CH * 1024) + c0 * 1024;
#pragma unroll
    for (int h = 0; h < S::BCH; ++h) {
      const int c2 = WM == 1 ? h : wm;
      copy16(tile + c2 * 1024, (uint32_t)(lane * 16), lds_addr(slot + S::B + ((wn * NT + n) * 2 + c2) * 1024));
    }
  }
  if (S::SA_RING) {
    if (wv < S::SW) {
      const int64_t ks = kt + 1 < p.KT ? kt + 1 : p.KT - 1;
      const uint32_t dst = lds_addr(sa_ring + ((kt + 1) % 3) * S::RING_ENTRY + (4 * MT * j + 16 * wv) * 16);
      if (ks == p.KT - 1 && p.K % kTileK != 0) copy4(static_cast<const uint8_t*>(p.sa), L.sa_last[j], dst);
      else copy4(static_cast<const uint8_t*>(p.sa) + ks * 4 * p.sa_ss, L.sa_piece[j], dst);
    }
  } else if (wv < S::SW) {  // activation scales of the 16 MT rows (row = t of the scale waves)
    if (!BLOCK)  // E8M0 bytes of blocks 4t .. 4t + 3
      copy4(static_cast<const uint8_t*>(p.sa) + t * p.sa_ss, L.sa_off, lds_addr(slot + S::SA + wv * 256));
    else  // fp32 scale of K128 group t (column-major [K/128, M])
      copy4(static_cast<const uint8_t*>(p.sa) + t * 4 * p.M, L.sa_off, lds_addr(slot + S::SA + wv * 256));
  }
  if (!BLOCK) {
#pragma unroll
    for (int n = 0; n < NT; ++n)
      if (WM == 1 || NT == 1 || (n & 1) == wm)
        copy4(L.sw_tile[n] + kt * 256, (uint32_t)(lane * 4), lds_addr(slot + S::SB + (wn * NT + n) * 256));
  }
}

// Operands of one K128 stage, read from its ring slot into registers.
template <int MT, int NT, bool BLOCK>
struct WideRegs {
  v8i a[MT];         // A fragment of m-tile i
  uint32_t sa[MT];   // MX: E8M0 of the lane's block (row r of m-tile i, block q of the slice)
  float4 s4[MT];     // block-FP8: fp32 activation scales of the lane's four output rows of m-tile i
  v8i b[NT];         // B fragment of the wave's n-tile n
  uint32_t sb[NT];   // MX: E8M0 of the lane's weight row, block q of the slice
  float sbv;         // block-FP8: the stage's weight block scale
};

// Read stage operands (slice j of its super-tile) from a slot: B fragments
// and scales first, then the MT A fragments in MFMA order.
template <int FMT, int MT, int NT, bool BLOCK, int WM>
__device__ __forceinline__ void wide_read(const uint8_t* slot, const uint8_t* sa_entry, int j, int wv, int lane,
                                          int q, int r, WideRegs<MT / WM, NT, BLOCK>& x) {
  using S = WideSlot<MT, NT, BLOCK, WM>;
  constexpr int MTW = MT / WM;
  const int wn = WM == 1 ? wv : wv & 3, i0 = WM == 1 ? 0 : (wv >> 2) * MTW;
  // FP6: the slice's 24 bytes start at byte 0 (even j) or 8 (odd j) of the first chunk
  const int odd = j & 1;
  const int o0 = 8 * odd, o1 = odd ? 1024 : 8, o2 = odd ? 1032 : 1024;
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const uint8_t* base = slot + S::B + (wn * NT + n) * 2048 + lane * 16;
    if (FMT == kE4M3) {
      const uint4 lo = *reinterpret_cast<const uint4*>(base);
      const uint4 hi = *reinterpret_cast<const uint4*>(base + 1024);
      x.b[n] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    } else {
      const uint2 d0 = *reinterpret_cast<const uint2*>(base + o0);
      const uint2 d1 = *reinterpret_cast<const uint2*>(base + o1);
      const uint2 d2 = *reinterpret_cast<const uint2*>(base + o2);
      x.b[n] = v8i{(int)d0.x, (int)d0.y, (int)d1.x, (int)d1.y, (int)d2.x, (int)d2.y, 0, 0};
    }
    if (!BLOCK) x.sb[n] = slot[S::SB + (wn * NT + n) * 256 + lane * 4 + j];  // byte j: slice j
  }
#pragma unroll
  for (int i = 0; i < MTW; ++i) {
    const int gi = i0 + i;  // the wave's i-th m-tile within the workgroup tile
    const uint8_t* row = slot + S::A + gi * 2048 + (r >> 3) * 1024 + (r & 7) * 128;
    const int sw = a_swz(r);
    const uint4 lo = *reinterpret_cast<const uint4*>(row + 16 * (q ^ sw));        // K 16 q ..
    const uint4 hi = *reinterpret_cast<const uint4*>(row + 16 * ((q + 4) ^ sw));  // K 64 + 16 q ..
    x.a[i] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    if (S::SA_RING) x.sa[i] = sa_entry[(16 * gi + r) * 16 + 4 * j + q];
    else if (!BLOCK) x.sa[i] = slot[S::SA + (16 * gi + r) * 4 + q];
    else x.s4[i] = *reinterpret_cast<const float4*>(slot + S::SA + (16 * gi + 4 * q) * 4);
  }
}

// The MT x NT MFMAs of one stage, from registers.  The E8M0 scales are single
// bytes (op_sel 0), since the slice index is not a compile-time value under a
// 3-slot ring.
template <int FMT, int MT, int NT, bool BLOCK>
__device__ __forceinline__ void wide_mfma(const WideRegs<MT, NT, BLOCK>& x, v4f (&acc)[MT][NT]) {
  if (!BLOCK) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[i][n] = mfma_step<FMT, 0>(x.a[i], x.b[n], acc[i][n], x.sa[i], x.sb[n]);
  } else {
    // block-FP8: each K128 product is folded with fma(raw, sa * sb, acc); the raw
    // products of m-tile i + 1 are issued before the folds of m-tile i, so no
    // fold waits on the MFMA just issued
    v4f raw[2][NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) raw[0][n] = mfma_raw<FMT>(x.a[0], x.b[n]);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      if (i + 1 < MT) {
#pragma unroll
        for (int n = 0; n < NT; ++n) raw[(i + 1) & 1][n] = mfma_raw<FMT>(x.a[i + 1], x.b[n]);
      }
      const float fs[4] = {x.s4[i].x * x.sbv, x.s4[i].y * x.sbv, x.s4[i].z * x.sbv, x.s4[i].w * x.sbv};
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][n][e] = __builtin_fmaf(raw[i & 1][n][e], fs[e], acc[i][n][e]);
    }
  }
}

// Scheduling groups for one step (MX): each MFMA followed by its share of the
// next stage's LDS reads.  (Block-FP8 steps are left to the default schedule,
// which measured faster than any grouping of their scale folds.)
template <int FMT, int MT, int NT, bool BLOCK>
__device__ __forceinline__ void wide_interleave() {
  if (!BLOCK) {
    constexpr int kMfma = MT * NT;
    constexpr int kReads = 2 * MT + MT + (FMT == kE4M3 ? 2 * NT : 3 * NT) + NT;
    constexpr int kPer = (kReads + kMfma - 1) / kMfma;
#pragma unroll
    for (int k = 0; k < kMfma; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);     // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, kPer, 0);  // LDS reads
    }
  }
}

// Wait for this wave's copies of one stage: the copies of the `later` (at most
// L) stages issued after it (C per stage, C + 1 for waves 0 and 1) may stay in
// flight.
template <int C, int L>
__device__ __forceinline__ void wide_wait(int later, bool scales) {
  if constexpr (L == 0) {
    wait_vm<0>();
  } else {
    if (later >= L) {
      if (scales) wait_vm<L * (C + 1)>();
      else wait_vm<L * C>();
    } else {
      wide_wait<C, L - 1>(later, scales);
    }
  }
}

// RNE binary32 pair -> packed bf16 pair (v_cvt_pk_bf16_f32), NaN -> 0x7FC0 as f32_to_bf16.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  typedef float f2 __attribute__((ext_vector_type(2)));
  uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, bf2));
  if (lo != lo) u = (u & 0xFFFF0000u) | 0x7FC0u;
  if (hi != hi) u = (u & 0x0000FFFFu) | 0x7FC00000u;
  return u;
}

}  // namespace

struct WideGrid {
  int64_t mblocks;       // dense: ceil(M / 16 MT); grouped: bound on sum_e ceil(rows_e / 16 MT)
  int64_t nblocks;       // ceil(N / (64 NT))
  int64_t kt_per_split;  // 512-wide super-tiles per split
  int64_t num_experts;   // grouped only
  int64_t tile0, tiles;  // dense: this launch covers output tiles [tile0, tile0 + tiles) (tile = nb * mblocks + mb)
  // dense, one-launch hybrid: after its whole-K tile (tiles [0, tiles), bf16 out) workgroup
  // L also runs unit L < rem_tiles * S2 of the remainder: tile rem_tile0 + L % rem_tiles,
  // K split L / rem_tiles of kt2 super-tiles, into compact partials
  int64_t rem_tile0, rem_tiles, kt2;
  int S2;
};

// One output tile: rows [row_base, hi) of m-block rows (hi bounds the valid rows
// of a grouped expert), n-block nb, K split `split`; w / sw are the expert's
// weights.  The ring and the scale ring are the workgroup's LDS.
template <int FMT, int MT, int NT, bool BLOCK, bool GROUPED, int WM>
__device__ __forceinline__ void wide_tile(const GemmParams& p, int64_t kps, int64_t row_base, int64_t hi,
                                          const uint8_t* w, const uint8_t* sw, int64_t nb, int64_t split,
                                          float* pdst, uint8_t* ring, uint8_t* sa_ring, float* sb_stage,
                                          int t, int lane, int wv, int r, int q) {
  using S = WideSlot<MT, NT, BLOCK, WM>;
  constexpr int C = S::COPIES;
  constexpr int BM = 16 * MT, MTW = MT / WM;
  const int wn = WM == 1 ? wv : wv & 3, wm = WM == 1 ? 0 : wv >> 2;
  auto a_row = [&](int64_t row) -> int64_t {
    if (row >= hi) row = hi - 1;  // padding rows copy a valid row; their outputs are not stored
    return (GROUPED && p.row_index) ? (int64_t)(p.row_index[row] / p.row_div) : row;
  };
  const int64_t ntiles_total = (p.N + 15) / 16;
  const int64_t nt_wave = (nb * 4 + wn) * NT;
  constexpr int CH = FmtTraits<FMT>::CH;
  WideLanes<MT, NT, WM> L;
#pragma unroll
  for (int u = 0; u < S::ACH; ++u) {
    const int c = S::ACH * wv + u;               // the A chunk: m-tile c / 2, rows 8 (c % 2) .. + 7
    const int cr = 8 * (c & 1) + (lane >> 3);  // the m-tile row this lane copies
    L.a_off[u] = (uint32_t)(a_row(row_base + (c >> 1) * 16 + cr) * p.lda + 16 * ((lane & 7) ^ a_swz(cr)));
  }
  // the scale waves' threads t < BM copy row t
  L.sa_off = (uint32_t)(BLOCK ? 4 * a_row(row_base + (t & (BM - 1))) : sa_row_offset(p, a_row(row_base + (t & (BM - 1)))));
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // dword (lane % 4) of the super-tile's four slice dwords of its row; a half last
    // super-tile (K % 512 = 256) clamps the slice inside K
    const int64_t srow = sa_row_offset(p, a_row(row_base + 4 * MT * j + 16 * (wv % S::SW) + (lane >> 2)));
    L.sa_piece[j] = (uint32_t)(srow + (lane & 3) * p.sa_ss);
    const int64_t last = 4 * (p.KT - 1) + (lane & 3);
    L.sa_last[j] = (uint32_t)(srow + (last < p.K / 128 - 1 ? last : p.K / 128 - 1) * p.sa_ss);
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int64_t nt = nt_wave + n < ntiles_total ? nt_wave + n : ntiles_total - 1;
    L.w_tile[n] = w + nt * p.KT * (CH * 1024);
    L.sw_tile[n] = sw + nt * p.KT * 256;
  }
  const int64_t T = p.K / 128;
  const int64_t tb = split * kps * 4;
  const int64_t te = tb + kps * 4 < T ? tb + kps * 4 : T;

  if (BLOCK) {
    // The wave's weight block scales of this split, copied into its LDS row (64 per
    // global->LDS copy) ahead of the stage copies, so the first stage's wait covers them.
    // Read inside the loop from global memory they would be the compiler's own vector
    // loads, which it waits for with vmcnt counts that include the stage copies (every
    // step would drain the ring); loaded into registers here, they cost a memory round
    // trip before the first copy is issued.
    const int64_t nt0 = nt_wave < ntiles_total ? nt_wave : ntiles_total - 1;
    const float* sbp = static_cast<const float*>(p.sw) + (nt0 * 16 / 128) * (p.K / 128) + tb;
    const int n_sb = (int)(te - tb);
    for (int c = 0; c < n_sb; c += 64) {  // lanes past the split re-read its last scale
      const int i = c + lane < n_sb ? c + lane : n_sb - 1;
      copy4(reinterpret_cast<const uint8_t*>(sbp), (uint32_t)(i * 4), lds_addr(reinterpret_cast<uint8_t*>(sb_stage + c)));
    }
  }

  v4f acc[MTW][NT];
#pragma unroll
  for (int i = 0; i < MTW; ++i)
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[i][n] = v4f{0.f, 0.f, 0.f, 0.f};

  // prologue: the scale ring entry of the first super-tile
  if (S::SA_RING && tb < te && wv < S::SW) {
    const bool half = (tb >> 2) == p.KT - 1 && p.K % kTileK != 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t dst = lds_addr(sa_ring + ((tb >> 2) % 3) * S::RING_ENTRY + (4 * MT * j + 16 * wv) * 16);
      if (half) copy4(static_cast<const uint8_t*>(p.sa), L.sa_last[j], dst);
      else copy4(static_cast<const uint8_t*>(p.sa) + (tb >> 2) * 4 * p.sa_ss, L.sa_piece[j], dst);
    }
  }
  if constexpr (GROUPED) {
    // Two workgroups per CU, each with a two-slot ring and one register set: step tt
    // waits for its own copies of stage tt (issued in the step before, the last ones
    // in flight), a barrier hands stage tt to every wave and frees the slot read in
    // the step before, stage tt + 1 is copied into it, then stage tt is read and
    // multiplied.  The other workgroup's steps run while this one waits on LDS
    // reads, copies or its prologue and epilogue.
    constexpr int R = kWideGroupedSlots;
    static_assert(4 % R == 0, "the four steps below rotate the slots");
    if (tb < te) wide_copy<FMT, MT, NT, BLOCK, WM>(p, ring, tb, wv, lane, L, sa_ring);
    WideRegs<MTW, NT, BLOCK> x;
#define MXL_WIDE_STEP2(I_)                                                                              \
  {                                                                                                   \
    const int64_t tt = t0 + I_;                                                                       \
    if (tt < te) {                                                                                    \
      wait_vm<0>();                                                                                   \
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");                                            \
      wide_barrier();                                                                                 \
      if (tt + 1 < te)                                                                                \
        wide_copy<FMT, MT, NT, BLOCK, WM>(p, ring + ((I_ + 1) % R) * S::BYTES, tt + 1, wv, lane, L, sa_ring); \
      wide_read<FMT, MT, NT, BLOCK, WM>(ring + (I_ % R) * S::BYTES, sa_ring + ((tt >> 2) % 3) * S::RING_ENTRY, \
                                        (int)(tt & 3), wv, lane, q, r, x);                           \
      if (BLOCK) x.sbv = sb_stage[tt - tb];                                                           \
      wide_mfma<FMT, MTW, NT, BLOCK>(x, acc);                                                         \
    }                                                                                                 \
  }
    // four steps per iteration: tb is a multiple of 4, so each step's slice index
    // (tt & 3) is a compile-time value and the per-slice lane offsets stay in registers
    for (int64_t t0 = tb; t0 < te; t0 += 4) {
      MXL_WIDE_STEP2(0)
      MXL_WIDE_STEP2(1)
      MXL_WIDE_STEP2(2)
      MXL_WIDE_STEP2(3)
    }
#undef MXL_WIDE_STEP2
  } else if (tb < te) {
    constexpr int R = S::SLOTS;
    // prologue: stages tb .. tb + R - 1 fill the ring; stage tb is read into registers
#pragma unroll
    for (int k = 0; k < R; ++k)
      if (tb + k < te) wide_copy<FMT, MT, NT, BLOCK, WM>(p, ring + k * S::BYTES, tb + k, wv, lane, L, sa_ring);
    wide_wait<C, R - 1>((int)(te - 1 - tb < R - 1 ? te - 1 - tb : R - 1), wv < S::SW);
    wide_barrier();
    WideRegs<MTW, NT, BLOCK> x0, x1;
    wide_read<FMT, MT, NT, BLOCK, WM>(ring, sa_ring + ((tb >> 2) % 3) * S::RING_ENTRY, (int)(tb & 3), wv, lane, q, r,
                                  x0);
    if (BLOCK) x0.sbv = sb_stage[0];

// Step tt = t0 + I (ring slot I % R): wait for stage tt + 1 and for this wave's
// reads of stage tt, barrier (every wave holds stage tt in registers, so its slot
// is free), copy stage tt + R into that slot, then the MFMAs of stage tt with the
// LDS reads of stage tt + 1 (into the other register set) interleaved between
// them: issued as one block, the reads would stall the wave's in-order issue on
// the LDS queue and the MFMAs would only start once the last read is queued.
// In the last step the reads fetch a stale slot and are never used.
#define MXL_WIDE_STEP(I_, CUR_, NXT_)                                                                 \
  {                                                                                                 \
    const int64_t tt = t0 + I_;                                                                     \
    if (tt < te) {                                                                                  \
      if (tt + 1 < te) {                                                                            \
        const int64_t later = te - 2 - tt < R - 2 ? te - 2 - tt : R - 2;                            \
        wide_wait<C, R - 2>((int)later, wv < S::SW);                                                  \
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");                                          \
        wide_barrier();                                                                             \
        if (tt + R < te) wide_copy<FMT, MT, NT, BLOCK, WM>(p, ring + ((I_) % R) * S::BYTES, tt + R, wv, lane, L, sa_ring); \
      }                                                                                             \
      wide_read<FMT, MT, NT, BLOCK, WM>(ring + ((I_ + 1) % R) * S::BYTES,                           \
                                    sa_ring + (((tt + 1) >> 2) % 3) * S::RING_ENTRY,            \
                                (int)((tt + 1) & 3), wv, lane, q, r, NXT_);                         \
      if (BLOCK) NXT_.sbv = sb_stage[(tt + 1 < te ? tt + 1 : tt) - tb];                             \
      wide_mfma<FMT, MTW, NT, BLOCK>(CUR_, acc);                                                    \
      wide_interleave<FMT, MTW, NT, BLOCK>();                                                       \
    }                                                                                               \
  }

    if (R == 4) {
      for (int64_t t0 = tb; t0 < te; t0 += 4) {
        MXL_WIDE_STEP(0, x0, x1)
        MXL_WIDE_STEP(1, x1, x0)
        MXL_WIDE_STEP(2, x0, x1)
        MXL_WIDE_STEP(3, x1, x0)
      }
    } else {
      for (int64_t t0 = tb; t0 < te; t0 += 6) {
        MXL_WIDE_STEP(0, x0, x1)
        MXL_WIDE_STEP(1, x1, x0)
        MXL_WIDE_STEP(2, x0, x1)
        MXL_WIDE_STEP(3, x1, x0)
        MXL_WIDE_STEP(4, x0, x1)
        MXL_WIDE_STEP(5, x1, x0)
      }
    }
#undef MXL_WIDE_STEP
  }

  // Epilogue through LDS: the waves write their fp32 accumulators into a
  // row-major 16 MT x 64 NT tile (row stride padded by 4 floats, so the 64 lanes
  // of a write -- rows 4 q + e, column r -- hit 64 distinct banks), then all
  // threads store whole 16-byte pieces of output rows.  Lane-scattered 2-byte
  // stores straight from the accumulator layout would cost a store instruction
  // per 64 values with 64-bit address arithmetic for each.
  constexpr int TW = 64 * NT, ST = TW + 4;
  static_assert(BM * ST * 4 <= (GROUPED ? kWideGroupedSlots : S::SLOTS) * S::BYTES, "epilogue tile exceeds the ring");
  if (pdst) {
    // fp32 split partials go straight from the accumulators, in MFMA fragment order: the
    // tile's block at pdst holds fragment f = m-tile * 4 NT + n-tile as 64 lanes x 4
    // floats (lane (q, r): rows 4 q .. 4 q + 3, column r), so every store instruction
    // writes 1 KiB contiguously; the split reduce puts them in row order.  No LDS round
    // trip or barrier (rows past M hold the padding rows' sums; the reduce skips them).
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int i = 0; i < MTW; ++i) {
        const int f = (wm * MTW + i) * (4 * NT) + wn * NT + n;
        *reinterpret_cast<float4*>(pdst + (f * 64 + lane) * 4) =
            float4{acc[i][n][0], acc[i][n][1], acc[i][n][2], acc[i][n][3]};
      }
    return;
  }
  float* const tile = reinterpret_cast<float*>(ring);
  wide_barrier();  // every wave is past its last fragment reads
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int i = 0; i < MTW; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        tile[(16 * (wm * MTW + i) + 4 * q + e) * ST + 16 * (wn * NT + n) + r] = acc[i][n][e];
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  const int64_t col0 = nb * TW;
  // Tiles whose columns all lie inside N (rows are checked per piece) take batched
  // passes: a thread issues the LDS reads of up to eight pieces before their stores, so it
  // waits on LDS once per batch instead of once per piece.
  constexpr int kThreads = 64 * S::WAVES;
  static_assert((BM * TW / 4) % kThreads == 0 && (BM * TW / 8) % kThreads == 0, "epilogue pieces per thread");
  {  // output elements (out_bits: alpha, format, bias), 8 columns per piece
    const bool vec = p.ldc % 8 == 0 && (reinterpret_cast<uintptr_t>(p.out) & 15) == 0;
    // bf16 without scale or bias: paired conversions
    const bool plain = !p.out_f16 && p.alpha == 1.0f && !p.bias;
    if (vec && col0 + TW <= p.N) {
      constexpr int P = BM * (TW / 8) / kThreads;
#pragma unroll
      for (int k0 = 0; k0 < P; k0 += 8) {
        float4 v[8][2];
#pragma unroll
        for (int k = 0; k < 8 && k0 + k < P; ++k) {
          const int c = t + (k0 + k) * kThreads;
          const float* src = tile + (c / (TW / 8)) * ST + (c % (TW / 8)) * 8;
          v[k][0] = *reinterpret_cast<const float4*>(src);
          v[k][1] = *reinterpret_cast<const float4*>(src + 4);
        }
#pragma unroll
        for (int k = 0; k < 8 && k0 + k < P; ++k) {
          const int c = t + (k0 + k) * kThreads;
          const int rr = c / (TW / 8), cc = (c % (TW / 8)) * 8;
          float f[8] = {v[k][0].x, v[k][0].y, v[k][0].z, v[k][0].w, v[k][1].x, v[k][1].y, v[k][1].z, v[k][1].w};
          uint32_t h[4];
          if (plain) {
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = pack_bf16x2(f[2 * e], f[2 * e + 1]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              h[e] = (uint32_t)out_bits(p, f[2 * e], col0 + cc + 2 * e) |
                     ((uint32_t)out_bits(p, f[2 * e + 1], col0 + cc + 2 * e + 1) << 16);
          }
          if (row_base + rr < hi)
            *reinterpret_cast<uint4*>(p.out + (row_base + rr) * p.ldc + col0 + cc) = uint4{h[0], h[1], h[2], h[3]};
        }
      }
      return;
    }
    for (int c = t; c < BM * (TW / 8); c += 64 * S::WAVES) {
      const int rr = c / (TW / 8), cc = (c % (TW / 8)) * 8;
      const int64_t row = row_base + rr, col = col0 + cc;
      if (row >= hi || col >= p.N) continue;
      const float4 v0 = *reinterpret_cast<const float4*>(tile + rr * ST + cc);
      const float4 v1 = *reinterpret_cast<const float4*>(tile + rr * ST + cc + 4);
      float f[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
      uint32_t h[4];
      if (plain) {
#pragma unroll
        for (int k = 0; k < 4; ++k) h[k] = pack_bf16x2(f[2 * k], f[2 * k + 1]);
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int64_t c0 = col + 2 * k < p.N ? col + 2 * k : p.N - 1;
          const int64_t c1 = col + 2 * k + 1 < p.N ? col + 2 * k + 1 : p.N - 1;
          h[k] = (uint32_t)out_bits(p, f[2 * k], c0) | ((uint32_t)out_bits(p, f[2 * k + 1], c1) << 16);
        }
      }
      uint16_t* dst = p.out + row * p.ldc + col;
      if (vec && col + 8 <= p.N) {
        *reinterpret_cast<uint4*>(dst) = uint4{h[0], h[1], h[2], h[3]};
      } else {
        for (int k = 0; k < 8 && col + k < p.N; ++k) dst[k] = (uint16_t)(k & 1 ? h[k >> 1] >> 16 : h[k >> 1]);
      }
    }
  }
}

// Largest number of experts the grouped variant keeps in LDS.
constexpr int kWideMaxExperts = (int)kWideGroupedMaxExperts;

// The grouped variant runs two workgroups per CU (at most 256 registers per lane and
// half the LDS each).
template <int FMT, int MT, int NT, bool BLOCK, bool GROUPED, int WM = 1>
__global__ __launch_bounds__(256 * WM, GROUPED ? 2 : 1) void gemm_wide_kernel(GemmParams p, WideGrid g) {
  static_assert(WM == 1 || !GROUPED, "the grouped variant runs four waves");
  using S = WideSlot<MT, NT, BLOCK, WM>;
  constexpr int BM = 16 * MT;
  // the stage ring (dense: the LDS budget of one workgroup per CU; grouped: two slots);
  // after the last stage it holds the output tile of the epilogue
  __shared__ __attribute__((aligned(16))) uint8_t ring[(GROUPED ? kWideGroupedSlots : S::SLOTS) * S::BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t sa_ring[S::SA_RING ? 3 * S::RING_ENTRY : 16];
  // block-FP8: each wave's weight block scales of the tile's K range
  __shared__ float sb_lds[BLOCK ? 4 * kWideBlockStages : 1];
  const int t = threadIdx.x, lane = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int r = lane & 15, q = lane >> 4;

  if (!GROUPED) {
    // XCD-aware remap of the linear workgroup id: the m-blocks sharing a weight
    // slice run consecutively on one XCD (workgroup L runs on XCD L % 8)
    const int64_t G = gridDim.x, Lid = blockIdx.x;
    const int64_t xcd = Lid & 7, per = G >> 3, extra = G & 7;
    const int64_t logical = xcd * per + (xcd < extra ? xcd : extra) + (Lid >> 3);
    constexpr int TW = 64 * NT;
    // (the two waves of an n-group share its row: they copy the same scales to it)
    float* const sbw = sb_lds + (BLOCK ? (wv & 3) * kWideBlockStages : 0);
    const uint8_t* const sw = static_cast<const uint8_t*>(p.sw);
    if (g.rem_tiles == 0) {
      const int64_t local = logical % g.tiles, split = logical / g.tiles;
      const int64_t tile = g.tile0 + local;
      const int64_t mb = tile % g.mblocks, nb = tile / g.mblocks;
      // split partials: the tile's fragment-ordered block, [split][tile][BM x TW]
      float* const pdst = p.S == 1 ? nullptr : p.partial + (split * g.tiles + local) * BM * TW;
      wide_tile<FMT, MT, NT, BLOCK, GROUPED, WM>(p, g.kt_per_split, mb * BM, p.M, p.w, sw, nb, split, pdst, ring,
                                                 sa_ring, sbw, t, lane, wv, r, q);
      return;
    }
    // one-launch hybrid: the whole-K tile, then the remainder unit (if any)
    if (logical < g.tiles) {
      const int64_t mb = logical % g.mblocks, nb = logical / g.mblocks;
      wide_tile<FMT, MT, NT, BLOCK, GROUPED, WM>(p, g.kt_per_split, mb * BM, p.M, p.w, sw, nb, 0, nullptr, ring,
                                                 sa_ring, sbw, t, lane, wv, r, q);
    }
    if (logical < g.rem_tiles * g.S2) {
      const int64_t local = logical % g.rem_tiles, split = logical / g.rem_tiles;
      const int64_t tile = g.rem_tile0 + local;
      const int64_t mb = tile % g.mblocks, nb = tile / g.mblocks;
      __syncthreads();  // the first tile's epilogue reads of the ring are done
      wide_tile<FMT, MT, NT, BLOCK, GROUPED, WM>(p, g.kt2, mb * BM, p.M, p.w, sw, nb, split,
                                                 p.partial + (split * g.rem_tiles + local) * BM * TW, ring, sa_ring,
                                                 sbw, t, lane, wv, r, q);
    }
    return;
  }

  // Grouped: persistent workgroups.  The experts' BM-row block counts are
  // prefix-summed once per workgroup into LDS; each workgroup then walks the
  // tiles L = blockIdx, blockIdx + grid, ... of the routed (m-block x n-block)
  // grid, n-blocks fastest (the same XCD remap, so a workgroup stays on its XCD's
  // tiles), and finds its expert by a parallel search of the prefix.  Only the prefix
  // stays in LDS (two workgroups share a CU's LDS); a tile reads its expert's row range
  // from expert_offsets.
  __shared__ int32_t sh_pre[kWideMaxExperts + 1];   // m-blocks before expert e
  __shared__ int32_t sh_hit;
  const int E = (int)g.num_experts;
  // block counts per thread chunk, then a block-wide inclusive scan of the chunk sums
  // (in the ring, which holds no stage yet)
  const int chunk = (E + 255) / 256;
  const int e0 = t * chunk < E ? t * chunk : E, e1 = e0 + chunk < E ? e0 + chunk : E;
  int cnt = 0;
  for (int e = e0; e < e1; ++e)
    cnt += (int)((p.expert_offsets[e + 1] - p.expert_offsets[e] + BM - 1) / BM);
  int32_t* const sh_scan = reinterpret_cast<int32_t*>(ring);
  sh_scan[t] = cnt;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int v = t >= off ? sh_scan[t - off] : 0;
    __syncthreads();
    sh_scan[t] += v;
    __syncthreads();
  }
  int base = sh_scan[t] - cnt;  // exclusive prefix of this thread's chunk
  for (int e = e0; e < e1; ++e) {
    sh_pre[e] = base;
    base += (int)((p.expert_offsets[e + 1] - p.expert_offsets[e] + BM - 1) / BM);
  }
  if (t == 255) sh_pre[E] = sh_scan[255];
  __syncthreads();
  const int64_t total_mb = sh_pre[E];
  // the routed tiles only (the launch's m-block count is a bound): the XCD remap then
  // spreads them evenly, whatever the tile order
  const int64_t Gt = (total_mb < g.mblocks ? total_mb : g.mblocks) * g.nblocks;
  const int64_t per = Gt >> 3, extra = Gt & 7;
  for (int64_t Lid = blockIdx.x; Lid < Gt; Lid += gridDim.x) {
    const int64_t xcd = Lid & 7;
    const int64_t logical = xcd * per + (xcd < extra ? xcd : extra) + (Lid >> 3);
    // n-blocks fastest: an expert block's n-blocks are consecutive, so they run on one
    // XCD and its gathered activation rows are fetched into that L2 once
    const int64_t nb = logical % g.nblocks;
    const int64_t mb = logical / g.nblocks;
    if (mb >= total_mb) continue;  // beyond the routed m-blocks (uniform)
    if (t == 0) sh_hit = 0;
    __syncthreads();
    for (int e = t; e < E; e += 256)
      if (sh_pre[e] <= mb && mb < sh_pre[e + 1]) sh_hit = e;
    __syncthreads();
    const int e = __builtin_amdgcn_readfirstlane(sh_hit);
    const int64_t rb = p.expert_offsets[e] + (mb - sh_pre[e]) * BM, rhi = p.expert_offsets[e + 1];
    const uint8_t* we = p.w + e * p.w_expert_stride;
    const uint8_t* swe = static_cast<const uint8_t*>(p.sw) + e * p.sw_expert_stride;
    // a 128-row block with at most 64 routed rows (an expert's last block) runs the
    // 64-row tile path in the same ring: half the activation copies and MFMAs
    if (MT == 8 && __builtin_amdgcn_readfirstlane((int)(rhi - rb)) <= 64)
      wide_tile<FMT, (MT == 8 ? 4 : MT), NT, BLOCK, GROUPED, 1>(p, g.kt_per_split, rb, rhi, we, swe, nb, 0, nullptr,
                                                             ring, sa_ring, sb_lds, t, lane, wv, r, q);
    else
      wide_tile<FMT, MT, NT, BLOCK, GROUPED, 1>(p, g.kt_per_split, rb, rhi, we, swe, nb, 0, nullptr, ring, sa_ring,
                                             sb_lds, t, lane, wv, r, q);
    __syncthreads();  // the epilogue's LDS reads are done before the next tile's copies
  }
}

// Sum the split partials of output tiles [tile0, tile0 + tiles) in split order, then the
// output rounding (out_bits: alpha, format, bias; the split-K reduce's arithmetic).  The
// partials are fragment-ordered tile blocks, [split][tile - tile0][BM x TW]: fragment f =
// m-tile * (TW / 16) + n-tile of a block is 64 lanes x 4 floats, lane (q, r) holding rows
// 4 q .. 4 q + 3 of column r.  One thread per (tile, fragment, lane): its S float4 loads
// are contiguous across the wave, and each of its four rows gets one 2-byte store (sixteen
// lanes cover 32 contiguous bytes of a row).
#ifndef MXL_WIDE_MX_DENSE_ONLY
__global__ __launch_bounds__(256) void wide_tile_reduce_kernel(const float* __restrict__ partial,
                                                               const uint16_t* __restrict__ bias,
                                                               uint16_t* __restrict__ out, int64_t M, int64_t N,
                                                               int64_t ldc, int64_t mblocks, int64_t tile0,
                                                               int64_t tiles, int S, int BM, int TW, float alpha,
                                                               int f16) {
  const int64_t per_tile = (int64_t)BM * TW / 4;  // float4 items of a tile block
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= tiles * per_tile) return;
  const int64_t local = id / per_tile;
  const int item = (int)(id - local * per_tile), f = item >> 6, lane = item & 63;
  const int nts = TW / 16;
  const int64_t tile = tile0 + local, mb = tile % mblocks, nb = tile / mblocks;
  const int64_t row0 = mb * BM + 16 * (f / nts) + 4 * (lane >> 4), col = nb * TW + 16 * (f % nts) + (lane & 15);
  if (row0 >= M || col >= N) return;
  const float4* src = reinterpret_cast<const float4*>(partial) + local * per_tile + item;
  const int64_t stride = tiles * per_tile;  // float4s per split
  float4 acc = src[0];
  for (int k0 = 1; k0 < S; k0 += 8) {
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (k0 + u < S) v[u] = src[(int64_t)(k0 + u) * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (k0 + u < S) {
        acc.x += v[u].x; acc.y += v[u].y; acc.z += v[u].z; acc.w += v[u].w;
      }
  }
  const float a4[4] = {acc.x, acc.y, acc.z, acc.w};
  const bool b = bias != nullptr;
  const uint16_t bv = b ? bias[col] : (uint16_t)0;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (row0 + e < M) out[(row0 + e) * ldc + col] = out_bits(a4[e], alpha, f16, b, bv);
}
#endif  // MXL_WIDE_MX_DENSE_ONLY

#ifndef MXL_WIDE_MX_DENSE_ONLY
// ------------------------------------------------------------ configuration

namespace {

// The hybrid split of `tiles` whole-K tiles over `cus` workgroup slots: full
// rounds first, the remainder split in K as evenly as the CUs allow.  Returns
// false when there is no partial last round to balance.
bool wide_hybrid(int64_t tiles, int64_t KT, int64_t cus, WideConfig& c) {
  if (tiles <= cus || tiles % cus == 0 || KT < 2) return false;
  const int64_t rem = tiles % cus;
  int64_t s2 = cus / rem < KT ? cus / rem : KT;
  if (s2 < 2) return false;
  const int64_t per = (KT + s2 - 1) / s2;
  c.dp_tiles = tiles - rem;
  c.kt2 = per;
  c.S2 = (int)((KT + per - 1) / per);
  return c.S2 >= 2;
}

}  // namespace

// Stage cost model (clock cycles at 2.4 GHz, one workgroup per CU) fitted to
// measurements on MI355X: a K128 stage of a 128-row tile costs about
// 1200 + 900 NT cycles (the stage copies, not the MFMAs, set the pace); a
// 64-row tile copies half the activations and issues half the MFMAs.
static double wide_stage_cycles(int mt, int nt) { return mt == 8 ? 1200.0 + 900.0 * nt : 800.0 + 800.0 * nt; }
// the split reduce's launch and ramp, in cycles of the stage model
constexpr double kWideReduceCycles = 8000.0;

// Pick the workgroup tile (MT, NT), the K split and the hybrid split from the
// stage model; weights stream at ~5 TB/s; split partials cost a write and a
// read of their bytes at ~3 TB/s.
WideConfig wide_config(int64_t M, int64_t N, int64_t K, int fmt, const GemmOptions& o) {
  const int64_t KT = (K + kTileK - 1) / kTileK;
  const int mt_force = o.tile_m == 4 || o.tile_m == 8 ? o.tile_m : 0;
  if ((o.tile_n == 1 || o.tile_n == 2 || o.tile_n == 4) && o.splits >= 1) {  // explicit tile and split
    const int mt = mt_force ? mt_force : 8;
    const int64_t per = (KT + o.splits - 1) / o.splits;
    WideConfig c{o.tile_n, (int)((KT + per - 1) / per), per};
    c.MT = mt;
    c.WM = o.waves == 8 && mt == 8 ? 2 : 1;
    if (o.hybrid && o.splits == 1)
      wide_hybrid(((M + 16 * mt - 1) / (16 * mt)) * ((N + 64 * o.tile_n - 1) / (64 * o.tile_n)), KT, cu_count(), c);
    return c;
  }
  const int64_t cus = cu_count();
  WideConfig best{2, 1, KT};
  double best_cost = 1e300;
  const double wbytes = (double)N * K * (fmt == kE4M3 ? 1.0 : 0.75) + (double)N * K / 32;
  const double hbm = (wbytes + (double)M * K * 1.04) / (5.0e12 / 2.4e9);
  // dense problems keep 128-row tiles unless forced or M <= 64: measured on the c2/c3/c4
  // shapes at M >= 128, 64-row tiles were 2-30 % slower (half the MFMAs per stage for the
  // same weight copies); at M = 64 the half-empty 128-row tiles lost on all three (per-shape
  // sweep: 7 %, 18 %, 22 %)
  const int mts[2] = {8, 4};
  const int nts[3] = {4, 2, 1};
  const int mt_auto = M <= 64 ? 4 : 8;
  for (int mt : mts) {
    if (mt_force ? mt != mt_force : mt != mt_auto) continue;
    const int64_t MB = (M + 16 * mt - 1) / (16 * mt);
    for (int nt : nts) {
      if (mt == 4 && nt == 1) continue;  // not instantiated
      if (o.tile_n && nt != o.tile_n) continue;
      const int64_t NBk = (N + 64 * nt - 1) / (64 * nt);
      const int64_t tiles = MB * NBk;
      const double t_stage = wide_stage_cycles(mt, nt);
      // a forced split count is rounded to the admissible one of its super-tiles per split
      const int64_t s_only = o.splits >= 1 ? (KT + (KT + o.splits - 1) / o.splits - 1) / ((KT + o.splits - 1) / o.splits) : 0;
      for (int64_t s = 1; s <= KT; ++s) {
        const int64_t per = (KT + s - 1) / s;
        if ((KT + per - 1) / per != s || (s_only && s != s_only)) continue;
        const double rounds = (double)((tiles * s + cus - 1) / cus);
        const double compute = rounds * per * 4 * t_stage + 3000.0;
        // a K split writes and re-reads its partials and adds the reduce launch (about 4 µs
        // in a graph: MXFP8 2048 x 2048 at M = 512 ran 12.4 µs whole-K against 15.8 split)
        const double partial =
            s > 1 ? ((double)M * N * 4 * s * 2 + (double)M * N * 2) / (3.0e12 / 2.4e9) + kWideReduceCycles : 0.0;
        const double cost = (compute > hbm ? compute : hbm) + partial;
        if (cost < best_cost) {
          best_cost = cost;
          best = WideConfig{nt, (int)s, per};
          best.MT = mt;
        }
        WideConfig h{nt, 1, KT};
        h.MT = mt;
        if (s_only > 1 || (o.splits == 1 && !o.hybrid)) continue;  // a forced split excludes the hybrid
        // (64-wide tiles re-read the activations too often for extra rounds to pay off)
        if (s == 1 && nt >= 2 && wide_hybrid(tiles, KT, cus, h)) {
          // full rounds with one remainder unit after the tile, its partials' round trip and
          // the reduce launch
          const double rem = (double)(tiles - h.dp_tiles);
          const double compute_h =
              (double)(h.dp_tiles / cus) * KT * 4 * t_stage + (double)h.kt2 * 4 * t_stage + 6000.0;
          const double partial_h = rem * 16 * mt * 64 * nt * 4 * h.S2 * 2 / (3.0e12 / 2.4e9);
          const double cost_h = (compute_h > hbm ? compute_h : hbm) + partial_h;
          if (cost_h < best_cost) {
            best_cost = cost_h;
            best = h;
          }
        }
      }
    }
  }
  if (o.waves == 8 && best.MT == 8) best.WM = 2;
  return best;
}

int64_t wide_workspace_bytes(const WideConfig& c, int64_t M, int64_t N) {
  // fragment-ordered partial blocks of whole tiles (padding rows and columns included)
  const int64_t bm = 16 * c.MT;
  const int64_t tiles = ((M + bm - 1) / bm) * ((N + 64 * c.NT - 1) / (64 * c.NT));
  if (c.dp_tiles > 0) return (int64_t)c.S2 * (tiles - c.dp_tiles) * bm * 64 * c.NT * 4;
  return c.S > 1 ? (int64_t)c.S * tiles * bm * 64 * c.NT * 4 : 0;
}

bool wide_gemm_eligible(int64_t M, int64_t K) { return M >= 64 && K % 256 == 0 && M * K < (int64_t(1) << 32); }

#endif  // MXL_WIDE_MX_DENSE_ONLY

template <int FMT, int MT, bool BLOCK, bool GROUPED>
static hipError_t launch_wide_mt(const WideConfig& c, const GemmParams& p, const WideGrid& g, int64_t grid,
                                 hipStream_t s) {
  const dim3 gr((unsigned)grid), blk(256);
  if (c.WM == 2) {  // eight waves: dense 128-row tiles
    if constexpr (GROUPED || MT != 8) {
      return hipErrorInvalidValue;
    } else {
      const dim3 blk8(512);
      if (c.NT == 4) {
        // block-FP8 with four n-tiles per wave does not fit two waves' registers per SIMD
        if constexpr (BLOCK) return hipErrorInvalidValue;
        else hipLaunchKernelGGL((gemm_wide_kernel<FMT, 8, 4, false, false, 2>), gr, blk8, 0, s, p, g);
      } else if (c.NT == 2) {
        hipLaunchKernelGGL((gemm_wide_kernel<FMT, 8, 2, BLOCK, false, 2>), gr, blk8, 0, s, p, g);
      } else if (c.NT == 1) {
        hipLaunchKernelGGL((gemm_wide_kernel<FMT, 8, 1, BLOCK, false, 2>), gr, blk8, 0, s, p, g);
      } else {
        return hipErrorInvalidValue;
      }
      return hipGetLastError();
    }
  }
  if (c.NT == 4) {
    if constexpr (GROUPED) return hipErrorInvalidValue;  // the grouped variant runs NT <= 2 (LDS)
    else hipLaunchKernelGGL((gemm_wide_kernel<FMT, MT, 4, BLOCK, GROUPED>), gr, blk, 0, s, p, g);
  } else if (c.NT == 2) {
    hipLaunchKernelGGL((gemm_wide_kernel<FMT, MT, 2, BLOCK, GROUPED>), gr, blk, 0, s, p, g);
  } else if (c.NT == 1) {
    if constexpr (MT == 4) return hipErrorInvalidValue;  // 64 x 64 tiles are not instantiated
    else hipLaunchKernelGGL((gemm_wide_kernel<FMT, MT, 1, BLOCK, GROUPED>), gr, blk, 0, s, p, g);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int FMT, bool BLOCK, bool GROUPED>
static hipError_t launch_wide_fmt(const WideConfig& c, const GemmParams& p, const WideGrid& g, int64_t grid,
                                  hipStream_t s) {
  if (c.MT == 8) return launch_wide_mt<FMT, 8, BLOCK, GROUPED>(c, p, g, grid, s);
  if (c.MT == 4) return launch_wide_mt<FMT, 4, BLOCK, GROUPED>(c, p, g, grid, s);
  return hipErrorInvalidValue;
}

// The dense MX launches (gemm_wide_mx.hip compiles this file again with
// MXL_WIDE_MX_DENSE_ONLY for them alone, under its own scheduling flags; the block-FP8
// and grouped launches stay in this translation unit).
hipError_t launch_wide_mx_dense(int fmt, const WideConfig& c, const GemmParams& q, const WideGrid& gg, int64_t n,
                                hipStream_t s)
#ifdef MXL_WIDE_MX_DENSE_ONLY
{
  if (fmt == kE4M3) return launch_wide_fmt<kE4M3, false, false>(c, q, gg, n, s);
  if (fmt == kE2M3) return launch_wide_fmt<kE2M3, false, false>(c, q, gg, n, s);
  if (fmt == kE3M2) return launch_wide_fmt<kE3M2, false, false>(c, q, gg, n, s);
  return hipErrorInvalidValue;
}
#else
;

hipError_t launch_gemm_wide(int fmt, bool block, const WideConfig& c, const GemmParams& p, int64_t num_experts,
                            hipStream_t s) {
  const int64_t bm = 16 * c.MT;
  if (block && (c.kt_per_split * 4 > kWideBlockStages || c.kt2 * 4 > kWideBlockStages)) return hipErrorInvalidValue;
  WideGrid g{};
  g.nblocks = (p.N + 64 * c.NT - 1) / (64 * c.NT);
  g.kt_per_split = c.kt_per_split;
  g.num_experts = num_experts;
  int64_t grid;
  if (num_experts > 0) {
    g.mblocks = (p.M + bm - 1) / bm + num_experts;  // bound on the routed m-blocks
    grid = g.mblocks * g.nblocks;
    if (grid > 2 * cu_count()) grid = 2 * cu_count();  // persistent workgroups (two per CU) walk the tiles
    if (fmt == kE4M3) return launch_wide_fmt<kE4M3, false, true>(c, p, g, grid, s);
    if (fmt == kE2M3) return launch_wide_fmt<kE2M3, false, true>(c, p, g, grid, s);
    if (fmt == kE3M2) return launch_wide_fmt<kE3M2, false, true>(c, p, g, grid, s);
    return hipErrorInvalidValue;
  }
  g.mblocks = (p.M + bm - 1) / bm;
  g.tile0 = 0;
  g.tiles = g.mblocks * g.nblocks;
  auto dense = [&](const GemmParams& q, const WideGrid& gg, int64_t n) -> hipError_t {
    if (block) return fmt == kE4M3 ? launch_wide_fmt<kE4M3, true, false>(c, q, gg, n, s) : hipErrorInvalidValue;
    return launch_wide_mx_dense(fmt, c, q, gg, n, s);
  };
  const int64_t tw = 64 * c.NT;
  auto tile_reduce = [&](int64_t tile0, int64_t tiles, int S) -> hipError_t {
    const int64_t items = tiles * bm * tw / 4;
    wide_tile_reduce_kernel<<<dim3((unsigned)((items + 255) / 256)), 256, 0, s>>>(
        p.partial, p.bias, p.out, p.M, p.N, p.ldc, g.mblocks, tile0, tiles, S, (int)bm, (int)tw, p.alpha, p.out_f16);
    return hipGetLastError();
  };
  if (c.dp_tiles <= 0 || c.dp_tiles >= g.tiles) {
    // every tile in one launch, split in K into fragment-ordered partials when S > 1
    const hipError_t e = dense(p, g, g.tiles * c.S);
    if (e != hipSuccess || p.S == 1) return e;
    return tile_reduce(0, g.tiles, p.S);
  }
  // hybrid, one launch: workgroup L runs whole-K tile L (full rounds, bf16 out) and then
  // unit L of the remainder, split in K into compact partials (p.partial); their reduce
  // follows.  (With more than one full round some units run in later rounds' workgroups;
  // the last round still ends one unit after its tiles.)
  GemmParams q = p;
  q.S = 1;
  WideGrid gd = g;
  gd.tiles = c.dp_tiles;
  gd.rem_tile0 = c.dp_tiles;
  gd.rem_tiles = g.tiles - c.dp_tiles;
  gd.kt2 = c.kt2;
  gd.S2 = c.S2;
  const int64_t units = gd.rem_tiles * c.S2;
  hipError_t e = dense(q, gd, c.dp_tiles > units ? c.dp_tiles : units);
  if (e != hipSuccess) return e;
  return tile_reduce(gd.rem_tile0, gd.rem_tiles, c.S2);
}

#endif  // MXL_WIDE_MX_DENSE_ONLY

}  // namespace mxl
