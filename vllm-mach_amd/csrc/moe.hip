// MoE token sort and weighted combine for gfx950.
//
// Token sort: routes r = t * topk + k are grouped by expert id, keeping
// ascending r inside each expert (a stable counting sort), which yields
//   expert_offsets[E + 1]  exclusive prefix of per-expert route counts
//   sorted_routes[pos]     route at each sorted position
//   inverse[r]             sorted position of each route (-1 if dropped)
// Three passes over 1024-route chunks: per-chunk histograms (LDS atomics,
// order free), one workgroup scanning chunks and experts (the two in one
// workgroup when the histograms fit in LDS), then a pass that
// ranks each route inside its chunk (a ballot match of the expert id's bits inside the
// wavefront plus an LDS prefix over the chunk's 16 wavefronts) and scatters.  A single chunk
// (decode-sized steps) runs all three in one workgroup.
//
// Combine: out[t, h] = bf16(sum_k y[inverse[t*topk + k], h] * w[t, k]),
// each product rounded to binary32 and added in ascending k from zero.
#include "mx_common.h"

namespace mxl {

constexpr int kChunk = 1024;

// Routes of the same key in the earlier lanes of this wavefront (the rank of the lane's
// route among its expert's routes in the wavefront); key = the expert id, or E for a
// route whose expert is outside [0, E).  The lanes holding the same key are found one key
// bit at a time with a ballot -- a bit's ballot, or its complement where the lane's bit
// is 0, keeps the lanes that agree on it -- bit_width(E) ballots (9 for 256 experts)
// instead of 64 lane-by-lane comparisons; only wavefront-uniform control flow, so every
// lane takes part in every ballot.
__device__ __forceinline__ int same_expert_rank(int key, int E, int lane) {
  const int bits = 32 - __builtin_clz((unsigned)E);
  uint64_t same = ~0ull;
  for (int b = 0; b < bits; ++b) {
    const bool bit = (key >> b) & 1;
    const uint64_t on = __ballot(bit);
    same &= bit ? on : ~on;
  }
  return __popcll(same & ((1ull << lane) - 1ull));
}

__global__ __launch_bounds__(kChunk) void route_hist_kernel(const int32_t* __restrict__ ids, int64_t R, int E,
                                                           int32_t* __restrict__ chunk_counts) {
  extern __shared__ int32_t hist[];
  const int64_t c = blockIdx.x;
  for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
  __syncthreads();
  const int64_t r = c * kChunk + threadIdx.x;
  if (r < R) {
    const int32_t e = ids[r];
    if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) chunk_counts[c * E + e] = hist[e];
}

// One workgroup: chunk bases per expert (in place) and expert offsets.
__global__ __launch_bounds__(1024) void route_scan_kernel(int32_t* __restrict__ chunk_counts, int64_t C, int E,
                                                         int64_t* __restrict__ expert_offsets) {
  extern __shared__ int64_t tot[];  // [2][E]
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int64_t run = 0;
    for (int64_t c = 0; c < C; ++c) {
      const int32_t v = chunk_counts[c * E + e];
      chunk_counts[c * E + e] = (int32_t)run;
      run += v;
    }
    tot[e] = run;
  }
  __syncthreads();
  // inclusive Hillis-Steele scan over E values (ping-pong buffers)
  int src = 0;
  for (int d = 1; d < E; d <<= 1) {
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      int64_t v = tot[src * E + e];
      if (e >= d) v += tot[src * E + e - d];
      tot[(1 - src) * E + e] = v;
    }
    __syncthreads();
    src = 1 - src;
  }
  for (int e = threadIdx.x; e < E; e += blockDim.x) expert_offsets[e + 1] = tot[src * E + e];
  if (threadIdx.x == 0) expert_offsets[0] = 0;
}

__global__ __launch_bounds__(kChunk) void route_scatter_kernel(const int32_t* __restrict__ ids, int64_t R, int E,
                                                              const int32_t* __restrict__ chunk_base,
                                                              const int64_t* __restrict__ expert_offsets,
                                                              int32_t* __restrict__ sorted_routes,
                                                              int32_t* __restrict__ inverse) {
  extern __shared__ int32_t whist[];  // [kChunk / 64][E]
  const int64_t c = blockIdx.x;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  constexpr int W = kChunk / 64;
  for (int i = t; i < W * E; i += blockDim.x) whist[i] = 0;
  const int64_t r = c * kChunk + t;
  const int32_t e = r < R ? ids[r] : -1;
  const bool valid = e >= 0 && e < E;
  const int rank = same_expert_rank(valid ? e : E, E, lane);
  __syncthreads();
  if (valid) atomicAdd(&whist[w * E + e], 1);
  __syncthreads();
  for (int x = t; x < E; x += blockDim.x) {
    int32_t run = 0;
    for (int v = 0; v < W; ++v) {
      const int32_t n = whist[v * E + x];
      whist[v * E + x] = run;
      run += n;
    }
  }
  __syncthreads();
  if (r >= R) return;
  if (!valid) {
    inverse[r] = -1;
    return;
  }
  const int64_t pos = expert_offsets[e] + chunk_base[c * E + e] + whist[w * E + e] + rank;
  sorted_routes[pos] = (int32_t)r;
  inverse[r] = (int32_t)pos;
}

// Count and scan in one workgroup when the per-chunk histograms fit in LDS
// (C x E <= kCountScanMaxEntries, E <= 1024): the chunk histograms of route_hist_kernel
// (route ids loaded eight at a time, LDS atomics), then per expert the running chunk
// bases in chunk order and the exclusive offsets -- the values route_scan_kernel writes,
// in one launch instead of two and without its serial walk through global memory.
constexpr int kCountScanMaxEntries = 14336;
__global__ __launch_bounds__(kChunk) void route_count_scan_kernel(const int32_t* __restrict__ ids, int64_t R,
                                                                  int64_t C, int E,
                                                                  int32_t* __restrict__ chunk_base,
                                                                  int64_t* __restrict__ expert_offsets) {
  extern __shared__ int32_t lds[];
  int32_t* hist = lds;              // [C][E]
  int32_t* tot = lds + C * E;       // [2][E]
  const int t = threadIdx.x;
  for (int64_t i = t; i < C * E; i += kChunk) hist[i] = 0;
  __syncthreads();
  for (int64_t c0 = 0; c0 < C; c0 += 8) {
    int32_t e[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t r = (c0 + k) * kChunk + t;
      e[k] = (c0 + k < C && r < R) ? ids[r] : -1;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (e[k] >= 0 && e[k] < E) atomicAdd(&hist[(c0 + k) * E + e[k]], 1);
  }
  __syncthreads();
  for (int x = t; x < E; x += kChunk) {
    int32_t run = 0;
    for (int64_t c = 0; c < C; ++c) {
      const int32_t n = hist[c * E + x];
      chunk_base[c * E + x] = run;
      run += n;
    }
    tot[x] = run;
  }
  __syncthreads();
  int src = 0;  // inclusive scan of the totals (ping-pong)
  for (int d = 1; d < E; d <<= 1) {
    for (int x = t; x < E; x += kChunk) {
      int32_t v = tot[src * E + x];
      if (x >= d) v += tot[src * E + x - d];
      tot[(1 - src) * E + x] = v;
    }
    __syncthreads();
    src = 1 - src;
  }
  for (int x = t; x < E; x += kChunk) expert_offsets[x + 1] = tot[src * E + x];
  if (t == 0) expert_offsets[0] = 0;
}

// All routes in one chunk (R <= 1024, E <= 1024): the three passes in one
// workgroup -- per-wavefront expert counts in LDS, per-expert totals scanned into
// the offsets, then the same rank and scatter -- so a decode-sized step pays one
// launch.  The result is the multi-chunk path's (chunk base 0).
constexpr int kSingleMaxExperts = 1024;
// Largest expert count any route schedule launches: the scatter's (kChunk / 64) * E
// ints of LDS must fit gfx950's 160 KiB per workgroup.
constexpr int kRouteMaxExperts = 160 * 1024 / ((kChunk / 64) * (int)sizeof(int32_t));
static_assert(kRouteMaxExperts == 2560, "the documented expert limit");

// The single-chunk sort for route t (expert e, -1 if none): per-wavefront expert counts in
// LDS, per-expert totals scanned into the offsets, then the rank and scatter.  Called by
// every thread of a 1024-thread workgroup (t = threadIdx.x).
__device__ __forceinline__ void single_chunk_sort(int32_t e, int64_t R, int E, int64_t* __restrict__ expert_offsets,
                                                  int32_t* __restrict__ sorted_routes,
                                                  int32_t* __restrict__ inverse, int32_t* whist,
                                                  int32_t (*tot)[kSingleMaxExperts]) {
  constexpr int W = kChunk / 64;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  for (int i = t; i < W * E; i += kChunk) whist[i] = 0;
  const bool valid = e >= 0 && e < E;
  const int rank = same_expert_rank(valid ? e : E, E, lane);
  __syncthreads();
  if (valid) atomicAdd(&whist[w * E + e], 1);
  __syncthreads();
  for (int x = t; x < E; x += kChunk) {  // per-wavefront bases and the expert's total
    int32_t run = 0;
    for (int v = 0; v < W; ++v) {
      const int32_t n = whist[v * E + x];
      whist[v * E + x] = run;
      run += n;
    }
    tot[0][x] = run;
  }
  __syncthreads();
  int src = 0;  // inclusive scan of the totals (ping-pong)
  for (int d = 1; d < E; d <<= 1) {
    for (int x = t; x < E; x += kChunk) {
      int32_t v = tot[src][x];
      if (x >= d) v += tot[src][x - d];
      tot[1 - src][x] = v;
    }
    __syncthreads();
    src = 1 - src;
  }
  for (int x = t; x < E; x += kChunk) expert_offsets[x + 1] = tot[src][x];
  if (t == 0) expert_offsets[0] = 0;
  if (t >= R) return;
  if (!valid) {
    inverse[t] = -1;
    return;
  }
  const int32_t pos = (e > 0 ? tot[src][e - 1] : 0) + whist[w * E + e] + rank;
  sorted_routes[pos] = t;
  inverse[t] = pos;
}

__global__ __launch_bounds__(kChunk) void route_single_kernel(const int32_t* __restrict__ ids, int64_t R, int E,
                                                             int64_t* __restrict__ expert_offsets,
                                                             int32_t* __restrict__ sorted_routes,
                                                             int32_t* __restrict__ inverse) {
  __shared__ int32_t whist[(kChunk / 64) * kSingleMaxExperts];
  __shared__ int32_t tot[2][kSingleMaxExperts];
  const int t = threadIdx.x;
  single_chunk_sort(t < R ? ids[t] : -1, R, E, expert_offsets, sorted_routes, inverse, whist, tot);
}

// ------------------------------------------------------------------ router
//
// softmax -> top-k -> (renormalize) from router logits, the selection of vLLM's fused
// top-k softmax that the reference's MoE layer runs before its experts (select_experts;
// src/vllm_mach/mxfp6/moe.py:142-152 fuses it into qwen35_router_quant_out): the k largest
// logits of a token (softmax is increasing, so they are its k largest probabilities), ties
// to the lower expert index, weights exp(x - max) / sum, the sum over the k selected
// (renormalize) or over every expert.  One wavefront per token, the token's logits spread
// over its lanes (expert i at lane i % 64, slot i / 64); each of the k rounds takes the
// wavefront maximum of (order key, lower index) over the logits not yet taken.

constexpr int kRouterSlots = kSingleMaxExperts / 64;  // logits per lane: E <= 1024
constexpr int kRouterMaxTopk = 64;

// Binary32 as an unsigned key in value order (-0 read as +0, so equal values tie; NaNs
// order outside the finite values by sign).
__device__ __forceinline__ uint32_t order_key(float x) {
  uint32_t u = f2u(x);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) { return u2f((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k); }

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, 64);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m, 64);
  return v;
}

// Route token t with the calling wavefront: ids / weights [t * topk + r] for r < topk;
// returns the lane's id (lane r < topk holds selection r, other lanes -1).
template <bool BF16>
__device__ __forceinline__ int32_t route_token(const void* __restrict__ logits, int64_t t, int E, int topk,
                                               bool renorm, int lane, int32_t* __restrict__ ids,
                                               float* __restrict__ weights) {
  uint32_t key[kRouterSlots];
#pragma unroll
  for (int j = 0; j < kRouterSlots; ++j) {
    const int i = lane + 64 * j;
    float x = 0.0f;
    if (i < E) x = BF16 ? bf16_to_f32(static_cast<const uint16_t*>(logits)[t * E + i])
                        : static_cast<const float*>(logits)[t * E + i];
    key[j] = i < E ? order_key(x) : 0u;
  }
  uint32_t taken = 0u;
  float my_x = 0.0f;
  int32_t my_id = -1;
  float top = 0.0f;
  for (int r = 0; r < topk; ++r) {
    uint64_t best = 0;  // (key, ~index): the larger key, then the lower index
#pragma unroll
    for (int j = 0; j < kRouterSlots; ++j) {
      const int i = lane + 64 * j;
      if (i < E && !((taken >> j) & 1u)) {
        const uint64_t c = ((uint64_t)key[j] << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i);
        best = c > best ? c : best;
      }
    }
    best = wave_max_u64(best);
    const int idx = (int)(0xFFFFFFFFu - (uint32_t)best);
    const float x = key_value((uint32_t)(best >> 32));
    if ((idx & 63) == lane) taken |= 1u << (idx >> 6);
    if (r == 0) top = x;
    if (lane == r) {
      my_x = x;
      my_id = idx;
    }
  }
  const float e = lane < topk ? mx_exp(my_x - top) : 0.0f;
  float denom;
  if (renorm) {
    denom = wave_sum(e);
  } else {
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < kRouterSlots; ++j)
      if (lane + 64 * j < E) part = part + mx_exp(key_value(key[j]) - top);
    denom = wave_sum(part);
  }
  if (lane < topk) {
    ids[t * topk + lane] = my_id;
    weights[t * topk + lane] = e / denom;
  }
  return my_id;
}

// T * topk <= 1024 routes and E <= 1024: routing and the token sort in one workgroup.
template <bool BF16>
__global__ __launch_bounds__(kChunk) void router_single_kernel(const void* __restrict__ logits, int64_t T, int E,
                                                              int topk, int renorm, int32_t* __restrict__ ids,
                                                              float* __restrict__ weights,
                                                              int64_t* __restrict__ expert_offsets,
                                                              int32_t* __restrict__ sorted_routes,
                                                              int32_t* __restrict__ inverse) {
  __shared__ int32_t whist[(kChunk / 64) * kSingleMaxExperts];
  __shared__ int32_t tot[2][kSingleMaxExperts];
  __shared__ int32_t sids[kChunk];
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  for (int64_t tok = w; tok < T; tok += kChunk / 64) {
    const int32_t id = route_token<BF16>(logits, tok, E, topk, renorm != 0, lane, ids, weights);
    if (lane < topk) sids[tok * topk + lane] = id;
  }
  __syncthreads();
  const int64_t R = T * topk;
  single_chunk_sort(t < R ? sids[t] : -1, R, E, expert_offsets, sorted_routes, inverse, whist, tot);
}

// Chunk c of 1024 routes = 1024 / topk whole tokens (topk divides 1024): route them and
// count the chunk's routes per expert (the histogram the scatter's chunk bases come from).
template <bool BF16>
__global__ __launch_bounds__(kChunk) void router_hist_kernel(const void* __restrict__ logits, int64_t T, int E,
                                                            int topk, int renorm, int32_t* __restrict__ ids,
                                                            float* __restrict__ weights,
                                                            int32_t* __restrict__ chunk_counts) {
  __shared__ int32_t hist[kSingleMaxExperts];
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int64_t c = blockIdx.x, per = kChunk / topk;
  for (int e = t; e < E; e += kChunk) hist[e] = 0;
  __syncthreads();
  for (int64_t k = w; k < per; k += kChunk / 64) {
    const int64_t tok = c * per + k;
    if (tok >= T) break;
    const int32_t id = route_token<BF16>(logits, tok, E, topk, renorm != 0, lane, ids, weights);
    if (lane < topk) atomicAdd(&hist[id], 1);
  }
  __syncthreads();
  for (int e = t; e < E; e += kChunk) chunk_counts[c * E + e] = hist[e];
}

// Every chunk's scatter from the chunk histograms (C x E <= kCountScanMaxEntries,
// E <= 1024): the workgroup sums the histograms of the chunks before its own (its chunk
// bases) and of all chunks (the expert totals, scanned into the offsets, which workgroup 0
// writes), then ranks and scatters its routes as route_scatter_kernel does.
__global__ __launch_bounds__(kChunk) void route_scan_scatter_kernel(const int32_t* __restrict__ ids, int64_t R,
                                                                   int64_t C, int E,
                                                                   const int32_t* __restrict__ chunk_counts,
                                                                   int64_t* __restrict__ expert_offsets,
                                                                   int32_t* __restrict__ sorted_routes,
                                                                   int32_t* __restrict__ inverse) {
  constexpr int W = kChunk / 64;
  __shared__ int32_t whist[W * kSingleMaxExperts];
  __shared__ int32_t base[kSingleMaxExperts];
  __shared__ int32_t tot[2][kSingleMaxExperts];
  const int64_t c = blockIdx.x;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  for (int x = t; x < E; x += kChunk) {
    int32_t before = 0, all = 0;
    for (int64_t cc = 0; cc < C; ++cc) {
      const int32_t n = chunk_counts[cc * E + x];
      if (cc < c) before += n;
      all += n;
    }
    base[x] = before;
    tot[0][x] = all;
  }
  for (int i = t; i < W * E; i += kChunk) whist[i] = 0;
  const int64_t r = c * kChunk + t;
  const int32_t e = r < R ? ids[r] : -1;
  const bool valid = e >= 0 && e < E;
  const int rank = same_expert_rank(valid ? e : E, E, lane);
  __syncthreads();
  if (valid) atomicAdd(&whist[w * E + e], 1);
  int src = 0;  // inclusive scan of the totals (ping-pong)
  for (int d = 1; d < E; d <<= 1) {
    __syncthreads();
    for (int x = t; x < E; x += kChunk) {
      int32_t v = tot[src][x];
      if (x >= d) v += tot[src][x - d];
      tot[1 - src][x] = v;
    }
    src = 1 - src;
  }
  __syncthreads();
  if (c == 0) {
    for (int x = t; x < E; x += kChunk) expert_offsets[x + 1] = tot[src][x];
    if (t == 0) expert_offsets[0] = 0;
  }
  for (int x = t; x < E; x += kChunk) {
    int32_t run = 0;
    for (int v = 0; v < W; ++v) {
      const int32_t n = whist[v * E + x];
      whist[v * E + x] = run;
      run += n;
    }
  }
  __syncthreads();
  if (r >= R) return;
  if (!valid) {
    inverse[r] = -1;
    return;
  }
  const int64_t pos = (e > 0 ? tot[src][e - 1] : 0) + base[e] + whist[w * E + e] + rank;
  sorted_routes[pos] = (int32_t)r;
  inverse[r] = (int32_t)pos;
}

// Routing only (shapes the fused schedules above do not take): ids and weights, sorted by
// mxl_moe_route afterwards.
template <bool BF16>
__global__ __launch_bounds__(256) void router_kernel(const void* __restrict__ logits, int64_t T, int E, int topk,
                                                     int renorm, int32_t* __restrict__ ids,
                                                     float* __restrict__ weights) {
  const int64_t tok = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok < T) route_token<BF16>(logits, tok, E, topk, renorm != 0, threadIdx.x & 63, ids, weights);
}

// One thread: 8 consecutive hidden columns of one token.
// addend (bf16 [T, H] or null): added to the fp32 sum after the routes, before the one rounding
__global__ __launch_bounds__(256) void moe_reduce_kernel(const uint16_t* __restrict__ y,
                                                         const float* __restrict__ topk_weights,
                                                         const int32_t* __restrict__ inverse, int64_t T, int topk,
                                                         int64_t H, const uint16_t* __restrict__ addend,
                                                         uint16_t* __restrict__ out) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_row = H / 8;
  if (id >= T * per_row) return;
  const int64_t t = id / per_row, h0 = (id - t * per_row) * 8;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  for (int k = 0; k < topk; ++k) {
    const int32_t p = inverse[t * topk + k];
    if (p < 0) continue;
    const float wk = topk_weights[t * topk + k];
    float v[8];
    bf16x8_to_f32(*reinterpret_cast<const uint4*>(y + (int64_t)p * H + h0), v);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float term = v[i] * wk;
      acc[i] = acc[i] + term;
    }
  }
  if (addend) {
    float v[8];
    bf16x8_to_f32(*reinterpret_cast<const uint4*>(addend + t * H + h0), v);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = acc[i] + v[i];
  }
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (uint32_t)f32_to_bf16(acc[2 * i]) | ((uint32_t)f32_to_bf16(acc[2 * i + 1]) << 16);
  *reinterpret_cast<uint4*>(out + t * H + h0) = make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace mxl

using namespace mxl;

extern "C" int64_t mxl_moe_route_workspace_bytes(int64_t T, int64_t topk, int64_t E) {
  const int64_t R = T * topk;
  const int64_t C = (R + kChunk - 1) / kChunk;
  return C * E * (int64_t)sizeof(int32_t);
}

extern "C" int mxl_moe_route(const int32_t* topk_ids, int64_t T, int64_t topk, int64_t E, int32_t* sorted_routes,
                             int64_t* expert_offsets, int32_t* inverse, void* workspace, int64_t workspace_bytes,
                             void* stream) {
  MXL_CHECK_ARG(T >= 0 && topk > 0 && E > 0, "mxl_moe_route: need T >= 0, topk > 0, E > 0");
  // route_scatter_kernel keeps one histogram per wavefront of a chunk in LDS:
  // (kChunk / 64) * E ints must fit gfx950's 160 KiB per workgroup
  MXL_CHECK_ARG(E <= kRouteMaxExperts, "mxl_moe_route: at most %d experts (E=%lld)", kRouteMaxExperts, (long long)E);
  const int64_t R = T * topk;
  const int64_t C = (R + kChunk - 1) / kChunk;
  MXL_CHECK_ARG(workspace_bytes >= mxl_moe_route_workspace_bytes(T, topk, E) && (C == 0 || workspace),
                "mxl_moe_route: workspace too small (%lld < %lld bytes)", (long long)workspace_bytes,
                (long long)mxl_moe_route_workspace_bytes(T, topk, E));
  hipStream_t s = (hipStream_t)stream;
  if (R <= kChunk && E <= kSingleMaxExperts) {  // one chunk: one launch
    route_single_kernel<<<1, kChunk, 0, s>>>(topk_ids, R, (int)E, expert_offsets, sorted_routes, inverse);
    MXL_CHECK_LAUNCH("mxl_moe_route(single)");
    return MXL_OK;
  }
  int32_t* counts = (int32_t*)workspace;
  if (C > 0 && C * E <= kCountScanMaxEntries && E <= 1024) {
    route_count_scan_kernel<<<1, kChunk, (C * E + 2 * E) * sizeof(int32_t), s>>>(topk_ids, R, C, (int)E, counts,
                                                                                  expert_offsets);
    MXL_CHECK_LAUNCH("mxl_moe_route(count_scan)");
  } else {
    if (C > 0) {
      route_hist_kernel<<<dim3((unsigned)C), kChunk, E * sizeof(int32_t), s>>>(topk_ids, R, (int)E, counts);
      MXL_CHECK_LAUNCH("mxl_moe_route(hist)");
    }
    route_scan_kernel<<<1, 1024, 2 * E * sizeof(int64_t), s>>>(counts, C, (int)E, expert_offsets);
    MXL_CHECK_LAUNCH("mxl_moe_route(scan)");
  }
  if (C > 0) {
    route_scatter_kernel<<<dim3((unsigned)C), kChunk, (kChunk / 64) * E * sizeof(int32_t), s>>>(
        topk_ids, R, (int)E, counts, expert_offsets, sorted_routes, inverse);
    MXL_CHECK_LAUNCH("mxl_moe_route(scatter)");
  }
  return MXL_OK;
}

// Router workspace: the chunk histograms of the two-launch schedule, or, for shapes the
// fused schedules do not take, mxl_moe_route's.
extern "C" int64_t mxl_moe_router_workspace_bytes(int64_t T, int64_t topk, int64_t E) {
  return mxl_moe_route_workspace_bytes(T, topk, E);
}

extern "C" int mxl_moe_router(const void* logits, int logits_bf16, int64_t T, int64_t E, int64_t topk,
                              int renormalize, float* topk_weights, int32_t* topk_ids, int32_t* sorted_routes,
                              int64_t* expert_offsets, int32_t* inverse, void* workspace, int64_t workspace_bytes,
                              void* stream) {
  MXL_CHECK_ARG(T >= 0 && E > 0 && E <= kSingleMaxExperts && topk > 0 && topk <= kRouterMaxTopk && topk <= E,
                "mxl_moe_router: need 0 < topk <= min(E, %d) and 0 < E <= %d (E=%lld topk=%lld)", kRouterMaxTopk,
                kSingleMaxExperts, (long long)E, (long long)topk);
  MXL_CHECK_ARG(logits_bf16 == 0 || logits_bf16 == 1, "mxl_moe_router: logits are fp32 (0) or bf16 (1)");
  const int64_t R = T * topk;
  const int64_t C = (R + kChunk - 1) / kChunk;
  MXL_CHECK_ARG(workspace_bytes >= mxl_moe_router_workspace_bytes(T, topk, E) && (C == 0 || workspace),
                "mxl_moe_router: workspace too small (%lld < %lld bytes)", (long long)workspace_bytes,
                (long long)mxl_moe_router_workspace_bytes(T, topk, E));
  hipStream_t s = (hipStream_t)stream;
  const int renorm = renormalize ? 1 : 0;
  if (R <= kChunk) {  // routing and the sort in one workgroup (also T = 0: the offsets)
    if (logits_bf16)
      router_single_kernel<true><<<1, kChunk, 0, s>>>(logits, T, (int)E, (int)topk, renorm, topk_ids, topk_weights,
                                                      expert_offsets, sorted_routes, inverse);
    else
      router_single_kernel<false><<<1, kChunk, 0, s>>>(logits, T, (int)E, (int)topk, renorm, topk_ids, topk_weights,
                                                       expert_offsets, sorted_routes, inverse);
    MXL_CHECK_LAUNCH("mxl_moe_router(single)");
    return MXL_OK;
  }
  int32_t* counts = (int32_t*)workspace;
  if (kChunk % topk == 0 && C * E <= kCountScanMaxEntries) {
    // chunks of whole tokens: routing with the chunk histograms, then the scan and scatter
    if (logits_bf16)
      router_hist_kernel<true><<<dim3((unsigned)C), kChunk, 0, s>>>(logits, T, (int)E, (int)topk, renorm, topk_ids,
                                                                    topk_weights, counts);
    else
      router_hist_kernel<false><<<dim3((unsigned)C), kChunk, 0, s>>>(logits, T, (int)E, (int)topk, renorm, topk_ids,
                                                                     topk_weights, counts);
    MXL_CHECK_LAUNCH("mxl_moe_router(hist)");
    route_scan_scatter_kernel<<<dim3((unsigned)C), kChunk, 0, s>>>(topk_ids, R, C, (int)E, counts, expert_offsets,
                                                                   sorted_routes, inverse);
    MXL_CHECK_LAUNCH("mxl_moe_router(scatter)");
    return MXL_OK;
  }
  const unsigned blocks = (unsigned)((T + 3) / 4);
  if (logits_bf16)
    router_kernel<true><<<blocks, 256, 0, s>>>(logits, T, (int)E, (int)topk, renorm, topk_ids, topk_weights);
  else
    router_kernel<false><<<blocks, 256, 0, s>>>(logits, T, (int)E, (int)topk, renorm, topk_ids, topk_weights);
  MXL_CHECK_LAUNCH("mxl_moe_router(route)");
  return mxl_moe_route(topk_ids, T, topk, E, sorted_routes, expert_offsets, inverse, workspace, workspace_bytes,
                       stream);
}

static int moe_reduce_common(const char* who, const void* routed_output, const float* topk_weights,
                             const int32_t* inverse, int64_t T, int64_t topk, int64_t H, const void* addend, void* out,
                             void* stream) {
  MXL_CHECK_ARG(T >= 0 && topk > 0 && H > 0 && H % 8 == 0, "%s: need H %% 8 == 0 (H=%lld)", who, (long long)H);
  MXL_CHECK_ARG(((uintptr_t)routed_output & 15) == 0 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)addend & 15) == 0,
                "%s: misaligned", who);
  if (T == 0) return MXL_OK;
  const int64_t n = T * (H / 8);
  moe_reduce_kernel<<<dim3((unsigned)((n + 255) / 256)), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)routed_output, topk_weights, inverse, T, (int)topk, H, (const uint16_t*)addend,
      (uint16_t*)out);
  MXL_CHECK_LAUNCH(who);
  return MXL_OK;
}

extern "C" int mxl_moe_reduce(const void* routed_output, const float* topk_weights, const int32_t* inverse, int64_t T,
                              int64_t topk, int64_t H, void* out, void* stream) {
  return moe_reduce_common("mxl_moe_reduce", routed_output, topk_weights, inverse, T, topk, H, nullptr, out, stream);
}

extern "C" int mxl_moe_reduce_add(const void* routed_output, const float* topk_weights, const int32_t* inverse,
                                  int64_t T, int64_t topk, int64_t H, const void* addend, void* out, void* stream) {
  MXL_CHECK_ARG(addend != nullptr, "mxl_moe_reduce_add: no addend");
  return moe_reduce_common("mxl_moe_reduce_add", routed_output, topk_weights, inverse, T, topk, H, addend, out,
                           stream);
}
