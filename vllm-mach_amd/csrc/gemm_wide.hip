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
// the MFMAs.  A slot holds
//   A    8 m-tiles x 2 KiB in MFMA fragment order: chunk (m-tile i, half h) has
//        at lane l = 16q + r the 16 bytes K [64 h + 16 q, +16) of row 16 i + r,
//        so a fragment is two lane-contiguous 16-byte LDS reads;
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
// on XCD L % 8) and hit its L2.  K splits (whole 512-wide super-tiles) write
// fp32 partials that a second kernel sums in split order.  The grouped variant
// walks experts' row ranges (expert_offsets) on device, so the launch needs no
// host-side counts.
#include <cstdio>
#include <cstdlib>

#include "gemm_common.h"

// the copies set M0 (the LDS base of a global->LDS load) themselves
#pragma clang diagnostic ignored "-Winline-asm"

namespace mxl {

namespace {

template <int NT, bool BLOCK>
struct WideSlot {
  static constexpr int A = 0;                          // 16 KiB
  static constexpr int B = 16 * 1024;                  // wave w: NT x 2 KiB at B + w NT 2 KiB
  static constexpr int SA = B + 4 * NT * 2048;         // 512 B, copied by waves 0 and 1
  static constexpr int SB = SA + 512;                  // wave w: NT x 256 B (MX)
  static constexpr int BYTES = SB + (BLOCK ? 0 : 4 * NT * 256);
  static constexpr int SLOTS = NT == 4 ? 3 : 4;        // 4 x 53 KiB would not fit the LDS
  // copies per wave per stage (waves 0 and 1 also copy the activation scales)
  static constexpr int COPIES = 4 + 2 * NT + (BLOCK ? 0 : NT);
};

typedef __attribute__((address_space(3))) uint8_t lds_u8;

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

template <int NT>
struct WideLanes {
  uint32_t a_off[2];  // row * lda + 16 q of the rows of m-tiles 2 wv, 2 wv + 1
  uint32_t sa_off;    // MX: row * K/32; block-FP8: 4 row  (row = t % 128)
  const uint8_t* w_tile[NT];  // wave-uniform: tile (ntile, 0) of each of the wave's n-tiles
  const uint8_t* sw_tile[NT];
};

// Copy K128 stage `t` (super-tile t / 4, slice j = t % 4) into a slot.
template <int FMT, int NT, bool BLOCK>
__device__ __forceinline__ void wide_copy(const GemmParams& p, uint8_t* slot, int64_t t, int wv, int lane,
                                          const WideLanes<NT>& L) {
  using S = WideSlot<NT, BLOCK>;
  constexpr int CH = FmtTraits<FMT>::CH;
  const int64_t kt = t >> 2;
  const int j = (int)(t & 3);
#pragma unroll
  for (int u = 0; u < 4; ++u) {  // A: m-tile 2 wv + u / 2, half u % 2
    const int i = 2 * wv + (u >> 1), hl = u & 1;
    copy16(p.a + t * 128 + 64 * hl, L.a_off[u >> 1], lds_addr(slot + S::A + (i * 2 + hl) * 1024));
  }
  // B: the two 1 KiB chunks of the tile that hold slice j (FP6: its 24 bytes per lane
  // straddle two chunks)
  const int c0 = FMT == kE4M3 ? 2 * j : (3 * j) >> 1;
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const uint8_t* tile = L.w_tile[n] + kt * (CH * 1024) + c0 * 1024;
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2)
      copy16(tile + c2 * 1024, (uint32_t)(lane * 16), lds_addr(slot + S::B + ((wv * NT + n) * 2 + c2) * 1024));
  }
  if (wv < 2) {  // activation scales of the 128 rows (row = t % 128 of waves 0, 1)
    if (!BLOCK)  // E8M0 bytes of blocks 4t .. 4t + 3
      copy4(static_cast<const uint8_t*>(p.sa) + t * 4, L.sa_off, lds_addr(slot + S::SA + wv * 256));
    else  // fp32 scale of K128 group t (column-major [K/128, M])
      copy4(static_cast<const uint8_t*>(p.sa) + t * 4 * p.M, L.sa_off, lds_addr(slot + S::SA + wv * 256));
  }
  if (!BLOCK) {
#pragma unroll
    for (int n = 0; n < NT; ++n)
      copy4(L.sw_tile[n] + kt * 256, (uint32_t)(lane * 4), lds_addr(slot + S::SB + (wv * NT + n) * 256));
  }
}

struct WideFrag {
  v8i a;
  uint32_t sd;  // MX: E8M0 dword of the fragment row (byte q is the lane's block)
  float4 s4;    // block-FP8: fp32 scales of the lane's four output rows
};

template <int NT, bool BLOCK>
__device__ __forceinline__ WideFrag wide_frag(const uint8_t* slot, int i, int lane, int q, int r) {
  using S = WideSlot<NT, BLOCK>;
  const uint8_t* fr = slot + S::A + i * 2048 + lane * 16;
  const uint4 lo = *reinterpret_cast<const uint4*>(fr);
  const uint4 hi = *reinterpret_cast<const uint4*>(fr + 1024);
  WideFrag x;
  x.a = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  if (!BLOCK) x.sd = *reinterpret_cast<const uint32_t*>(slot + S::SA + (16 * i + r) * 4);
  else x.s4 = *reinterpret_cast<const float4*>(slot + S::SA + (16 * i + 4 * q) * 4);
  return x;
}

// The 8 x NT MFMAs of one K128 stage (slice j of its super-tile).  The E8M0
// bytes are shifted into place (op_sel 0), since j is not a compile-time value
// under a 3-slot ring.  Fragment reads run one m-tile ahead of the MFMAs.
template <int FMT, int NT, bool BLOCK>
__device__ __forceinline__ void wide_compute(const uint8_t* slot, int j, float sbv, v4f (&acc)[8][NT], int wv,
                                             int lane, int q, int r) {
  using S = WideSlot<NT, BLOCK>;
  v8i bf[NT];
  uint32_t sb[NT];
  // FP6: the slice's 24 bytes start at byte 0 (even j) or 8 (odd j) of the first chunk
  const int odd = j & 1;
  const int o0 = 8 * odd, o1 = odd ? 1024 : 8, o2 = odd ? 1032 : 1024;
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const uint8_t* base = slot + S::B + (wv * NT + n) * 2048 + lane * 16;
    if (FMT == kE4M3) {
      const uint4 lo = *reinterpret_cast<const uint4*>(base);
      const uint4 hi = *reinterpret_cast<const uint4*>(base + 1024);
      bf[n] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    } else {
      const uint2 d0 = *reinterpret_cast<const uint2*>(base + o0);
      const uint2 d1 = *reinterpret_cast<const uint2*>(base + o1);
      const uint2 d2 = *reinterpret_cast<const uint2*>(base + o2);
      bf[n] = v8i{(int)d0.x, (int)d0.y, (int)d1.x, (int)d1.y, (int)d2.x, (int)d2.y, 0, 0};
    }
    if (!BLOCK) sb[n] = (*reinterpret_cast<const uint32_t*>(slot + S::SB + (wv * NT + n) * 256 + lane * 4) >> (8 * j)) & 0xFFu;
  }
  WideFrag cur = wide_frag<NT, BLOCK>(slot, 0, lane, q, r);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    WideFrag nxt;
    if (i < 7) nxt = wide_frag<NT, BLOCK>(slot, i + 1, lane, q, r);
    if (!BLOCK) {
      const uint32_t sa = (cur.sd >> (8 * q)) & 0xFFu;
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[i][n] = mfma_step<FMT, 0>(cur.a, bf[n], acc[i][n], sa, sb[n]);
    } else {
      const float fs[4] = {cur.s4.x * sbv, cur.s4.y * sbv, cur.s4.z * sbv, cur.s4.w * sbv};
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        const v4f raw = mfma_raw<FMT>(cur.a, bf[n]);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][n][e] = __builtin_fmaf(raw[e], fs[e], acc[i][n][e]);
      }
    }
    if (i < 7) cur = nxt;
  }
}

// Wait for this wave's copies of the current stage: the copies of the `later`
// stages issued after it (C per stage, C + 1 for waves 0 and 1) may stay in flight.
template <int C>
__device__ __forceinline__ void wide_wait(int later, bool scales) {
  if (scales) {
    if (later >= 2) wait_vm<2 * (C + 1)>();
    else if (later == 1) wait_vm<C + 1>();
    else wait_vm<0>();
  } else {
    if (later >= 2) wait_vm<2 * C>();
    else if (later == 1) wait_vm<C>();
    else wait_vm<0>();
  }
}

}  // namespace

struct WideGrid {
  int64_t mblocks;       // dense: ceil(M / 128); grouped: bound on sum_e ceil(rows_e / 128)
  int64_t nblocks;       // ceil(N / (64 NT))
  int64_t kt_per_split;  // 512-wide super-tiles per split
  int64_t num_experts;   // grouped only
};

template <int FMT, int NT, bool BLOCK, bool GROUPED>
__global__ __launch_bounds__(256) void gemm_wide_kernel(GemmParams p, WideGrid g) {
  using S = WideSlot<NT, BLOCK>;
  // separate objects per slot (the LDS budget of one workgroup per CU; with
  // three slots the fourth object is a 16-byte stub)
  __shared__ __attribute__((aligned(16))) uint8_t slot0[S::BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t slot1[S::BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t slot2[S::BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t slot3[S::SLOTS == 4 ? S::BYTES : 16];
  __shared__ int64_t sh_scan[256];
  __shared__ int64_t sh_grp[3];
  constexpr int C = S::COPIES;

  const int t = threadIdx.x, lane = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int r = lane & 15, q = lane >> 4;

  // XCD-aware remap of the linear workgroup id
  const int64_t G = gridDim.x, Lid = blockIdx.x;
  const int64_t xcd = Lid & 7, per = G >> 3, extra = G & 7;
  const int64_t logical = xcd * per + (xcd < extra ? xcd : extra) + (Lid >> 3);
  const int64_t mb = logical % g.mblocks;
  const int64_t rest = logical / g.mblocks;
  const int64_t nb = rest % g.nblocks;
  const int64_t split = rest / g.nblocks;

  int64_t row_base = mb * 128, hi = p.M;
  const uint8_t* w = p.w;
  const uint8_t* sw = static_cast<const uint8_t*>(p.sw);
  if (GROUPED) {
    // find the expert whose m-blocks contain global m-block `mb`
    const int64_t E = g.num_experts;
    const int64_t chunk = (E + 255) / 256;
    const int64_t e0 = t * chunk < E ? t * chunk : E, e1 = e0 + chunk < E ? e0 + chunk : E;
    int64_t cnt = 0;
    for (int64_t e = e0; e < e1; ++e) cnt += (p.expert_offsets[e + 1] - p.expert_offsets[e] + 127) / 128;
    sh_scan[t] = cnt;
    if (t == 0) sh_grp[0] = -1;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
      const int64_t v = t >= off ? sh_scan[t - off] : 0;
      __syncthreads();
      sh_scan[t] += v;
      __syncthreads();
    }
    int64_t base = sh_scan[t] - cnt;  // exclusive prefix
    if (mb >= base && mb < base + cnt) {
      for (int64_t e = e0; e < e1; ++e) {
        const int64_t lo_e = p.expert_offsets[e], hi_e = p.expert_offsets[e + 1];
        const int64_t nbk = (hi_e - lo_e + 127) / 128;
        if (mb < base + nbk) {
          sh_grp[0] = e;
          sh_grp[1] = lo_e + (mb - base) * 128;
          sh_grp[2] = hi_e;
          break;
        }
        base += nbk;
      }
    }
    __syncthreads();
    if (sh_grp[0] < 0) return;  // beyond the routed m-blocks (uniform)
    const int64_t e = __builtin_amdgcn_readfirstlane((int)sh_grp[0]);
    w += e * p.w_expert_stride;
    sw += e * p.sw_expert_stride;
    row_base = sh_grp[1];
    hi = sh_grp[2];
  }

  auto a_row = [&](int64_t row) -> int64_t {
    if (row >= hi) row = hi - 1;  // padding rows copy a valid row; their outputs are not stored
    return (GROUPED && p.row_index) ? (int64_t)(p.row_index[row] / p.row_div) : row;
  };
  const int64_t ntiles_total = (p.N + 15) / 16;
  const int64_t nt_wave = (nb * 4 + wv) * NT;
  constexpr int CH = FmtTraits<FMT>::CH;
  WideLanes<NT> L;
#pragma unroll
  for (int i = 0; i < 2; ++i) L.a_off[i] = (uint32_t)(a_row(row_base + (2 * wv + i) * 16 + r) * p.lda + 16 * q);
  L.sa_off = (uint32_t)(BLOCK ? 4 * a_row(row_base + (t & 127)) : a_row(row_base + (t & 127)) * (p.K / 32));  // t < 128 copy
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int64_t nt = nt_wave + n < ntiles_total ? nt_wave + n : ntiles_total - 1;
    L.w_tile[n] = w + nt * p.KT * (CH * 1024);
    L.sw_tile[n] = sw + nt * p.KT * 256;
  }
  const float* sbp = nullptr;
  if (BLOCK) {
    const int64_t nt0 = nt_wave < ntiles_total ? nt_wave : ntiles_total - 1;
    sbp = static_cast<const float*>(p.sw) + (nt0 * 16 / 128) * (p.K / 128);
  }

  const int64_t T = p.K / 128;
  const int64_t tb = split * g.kt_per_split * 4;
  const int64_t te = tb + g.kt_per_split * 4 < T ? tb + g.kt_per_split * 4 : T;

  v4f acc[8][NT];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[i][n] = v4f{0.f, 0.f, 0.f, 0.f};

  if (tb < te) {
    constexpr int R = S::SLOTS;
    // prologue: stages tb .. tb + R - 2
    wide_copy<FMT, NT, BLOCK>(p, slot0, tb, wv, lane, L);
    if (tb + 1 < te) wide_copy<FMT, NT, BLOCK>(p, slot1, tb + 1, wv, lane, L);
    if (R == 4 && tb + 2 < te) wide_copy<FMT, NT, BLOCK>(p, slot2, tb + 2, wv, lane, L);

// Step tt = t0 + I: wait for stage tt, barrier (the slot of tt - 1 is free),
// copy stage tt + R - 1 into it, then the stage's MFMAs.
#define MXL_WIDE_STEP(I_, SLOT_, NEXT_SLOT_)                                                       \
  {                                                                                               \
    const int64_t tt = t0 + I_;                                                                   \
    if (tt < te) {                                                                                \
      const int64_t later = te - 1 - tt < R - 2 ? te - 1 - tt : R - 2;                            \
      wide_wait<C>((int)later, wv < 2);                                                           \
      wide_barrier();                                                                             \
      if (tt + R - 1 < te) wide_copy<FMT, NT, BLOCK>(p, NEXT_SLOT_, tt + R - 1, wv, lane, L);     \
      wide_compute<FMT, NT, BLOCK>(SLOT_, (int)(tt & 3), BLOCK ? sbp[tt] : 0.f, acc, wv, lane, q, r); \
    }                                                                                             \
  }

    if (R == 4) {
      for (int64_t t0 = tb; t0 < te; t0 += 4) {
        MXL_WIDE_STEP(0, slot0, slot3)
        MXL_WIDE_STEP(1, slot1, slot0)
        MXL_WIDE_STEP(2, slot2, slot1)
        MXL_WIDE_STEP(3, slot3, slot2)
      }
    } else {
      for (int64_t t0 = tb; t0 < te; t0 += 3) {
        MXL_WIDE_STEP(0, slot0, slot2)
        MXL_WIDE_STEP(1, slot1, slot0)
        MXL_WIDE_STEP(2, slot2, slot1)
      }
    }
#undef MXL_WIDE_STEP
  }

  // epilogue: lane holds rows 4q + e, column r of each 16 x 16 tile
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int64_t nt = nt_wave + n;
    const int64_t col = nt * 16 + r;
    if (nt >= ntiles_total || col >= p.N) continue;
    const float bias = p.bias ? bf16_to_f32(p.bias[col]) : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t row = row_base + 16 * i + 4 * q + e;
        if (row >= hi) continue;
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

// ------------------------------------------------------------ configuration

namespace {

// Optional override "NT,S" (tuning runs only), e.g. MXL_WIDE_CONFIG=4,3.
bool wide_override(int& nt, int& s) {
  const char* v = std::getenv("MXL_WIDE_CONFIG");
  int o_nt = 0, o_s = 0;
  if (!v || std::sscanf(v, "%d,%d", &o_nt, &o_s) != 2 || (o_nt != 1 && o_nt != 2 && o_nt != 4) || o_s < 1) return false;
  nt = o_nt;
  s = o_s;
  return true;
}

}  // namespace

// Pick the n-tiles per wave and the K split from a time model fitted to
// measurements on MI355X (clock cycles at 2.4 GHz, one workgroup per CU): a
// K128 stage costs about 1200 + 900 NT cycles (the stage copies, not the
// MFMAs, set the pace); weights stream at ~5 TB/s; split partials cost a write
// and a read of M x N x 4 bytes per split at ~3 TB/s.
WideConfig wide_config(int64_t M, int64_t N, int64_t K, int fmt) {
  const int64_t KT = (K + kTileK - 1) / kTileK, MB = (M + 127) / 128;
  int o_nt, o_s;
  if (wide_override(o_nt, o_s)) {
    const int64_t per = (KT + o_s - 1) / o_s;
    return WideConfig{o_nt, (int)((KT + per - 1) / per), per};
  }
  WideConfig best{2, 1, KT};
  double best_cost = 1e300;
  const double wbytes = (double)N * K * (fmt == kE4M3 ? 1.0 : 0.75) + (double)N * K / 32;
  const double hbm = (wbytes + (double)M * K * 1.04) / (5.0e12 / 2.4e9);
  const int nts[3] = {4, 2, 1};
  for (int nt : nts) {
    const int64_t NBk = (N + 64 * nt - 1) / (64 * nt);
    const int64_t tiles = MB * NBk;
    for (int64_t s = 1; s <= KT; ++s) {
      const int64_t per = (KT + s - 1) / s;
      if ((KT + per - 1) / per != s) continue;
      const double rounds = (double)((tiles * s + 255) / 256);
      const double t_stage = 1200.0 + 900.0 * nt;
      const double compute = rounds * per * 4 * t_stage + 3000.0;
      const double partial = s > 1 ? ((double)M * N * 4 * s * 2 + (double)M * N * 2) / (3.0e12 / 2.4e9) : 0.0;
      const double cost = (compute > hbm ? compute : hbm) + partial;
      if (cost < best_cost) {
        best_cost = cost;
        best = WideConfig{nt, (int)s, per};
      }
    }
  }
  return best;
}

bool wide_gemm_eligible(int64_t M, int64_t K) {
  const char* v = std::getenv("MXL_WIDE_DISABLE");  // tuning runs only: compare with the older kernels
  return !(v && v[0] == '1') && M >= 64 && K % 256 == 0 && M * K < (int64_t(1) << 32);
}

template <int FMT, bool BLOCK, bool GROUPED>
static hipError_t launch_wide_fmt(const WideConfig& c, const GemmParams& p, const WideGrid& g, int64_t grid,
                                  hipStream_t s) {
  if (c.NT == 4) hipLaunchKernelGGL((gemm_wide_kernel<FMT, 4, BLOCK, GROUPED>), dim3((unsigned)grid), dim3(256), 0, s, p, g);
  else if (c.NT == 2) hipLaunchKernelGGL((gemm_wide_kernel<FMT, 2, BLOCK, GROUPED>), dim3((unsigned)grid), dim3(256), 0, s, p, g);
  else if (c.NT == 1) hipLaunchKernelGGL((gemm_wide_kernel<FMT, 1, BLOCK, GROUPED>), dim3((unsigned)grid), dim3(256), 0, s, p, g);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_gemm_wide(int fmt, bool block, const WideConfig& c, const GemmParams& p, int64_t num_experts,
                            hipStream_t s) {
  WideGrid g;
  g.nblocks = (p.N + 64 * c.NT - 1) / (64 * c.NT);
  g.kt_per_split = c.kt_per_split;
  g.num_experts = num_experts;
  int64_t grid;
  if (num_experts > 0) {
    g.mblocks = (p.M + 127) / 128 + num_experts;
    grid = g.mblocks * g.nblocks;
    if (fmt == kE4M3) return launch_wide_fmt<kE4M3, false, true>(c, p, g, grid, s);
    if (fmt == kE2M3) return launch_wide_fmt<kE2M3, false, true>(c, p, g, grid, s);
    if (fmt == kE3M2) return launch_wide_fmt<kE3M2, false, true>(c, p, g, grid, s);
    return hipErrorInvalidValue;
  }
  g.mblocks = (p.M + 127) / 128;
  grid = g.mblocks * g.nblocks * c.S;
  if (block) return fmt == kE4M3 ? launch_wide_fmt<kE4M3, true, false>(c, p, g, grid, s) : hipErrorInvalidValue;
  if (fmt == kE4M3) return launch_wide_fmt<kE4M3, false, false>(c, p, g, grid, s);
  if (fmt == kE2M3) return launch_wide_fmt<kE2M3, false, false>(c, p, g, grid, s);
  if (fmt == kE3M2) return launch_wide_fmt<kE3M2, false, false>(c, p, g, grid, s);
  return hipErrorInvalidValue;
}

}  // namespace mxl
