// libmxlinear_torch.so -- the reference's native operator names and schemas,
// registered over this library's C ABI (include/mxlinear.h), so that the
// reference's loaders can bind it where they load their own native libraries:
//
//   torch.ops.load_library(VLLM_MACH_BLOCK_FP8_LIBRARY)   src/vllm_mach/fp8/block_native.py:22-44
//   torch.ops.load_library(MXFP8_LIBRARY_PATH)            src/vllm_mach/mxfp8/native_backend.py:100-125
//   torch.ops.mxfp8_sm120.{gemm,gemm_from_float}_pdl,     src/vllm_mach/mxfp6/dense_mxfp8.py:54-95
//     mxfp6.quantize_mxfp8_pdl, mxfp8_sm120.dual_gemm_out native_backend.py:90-93
//   torch.ops.mach_fp8_activation.run                     native/fp8_activation/activation.cu:98-104
//   torch.ops.mxfp6.*                                     src/vllm_mach/mxfp6/dense.py:113-129,
//                                                         dense_mxfp8.py:40, fused_mlp.py:16-19,
//                                                         ar_norm.py:144-147
//
// Host code only (no kernels): every op validates its operands, then calls the
// C ABI on the current HIP stream of its device; a failing call raises with the
// library's message.  Weights reach these ops in the reference's logical
// layouts (E4M3 [N, K], packed FP6 [N, 3K/4], the 64-row duplicated block-FP8
// scales, swizzled E8M0 weight scales); the GEMMs read an MFMA-tiled copy made
// once per weight (the repack the reference does at load time) and cached,
// keyed by the weight's and scale's storage, invalidated when either tensor's
// version changes; an entry whose weight or scale storage has been freed is
// dropped by the next calls (each call checks a few entries, a cache miss all of
// them), so a freed weight's copy does not outlive it.  A cache miss or a
// workspace that must grow during HIP graph capture raises: warm every shape on
// the capture stream first, as the reference requires (native_backend.py:159-170).
#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>
#include <torch/library.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <map>
#include <mutex>
#include <optional>
#include <tuple>
#include <vector>

#include "mxlinear.h"

namespace {

constexpr int kE4M3 = 0, kE3M2 = 3;
constexpr int kFloorCarry175 = 0, kCeilDiv448 = 1;

hipStream_t stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

void check(int rc, const char* what) {
  TORCH_CHECK(rc == MXL_OK, what, " failed (", rc, "): ", mxl_last_error());
}

bool is_byte_dtype(const at::Tensor& t) {
  return t.scalar_type() == at::kByte || t.scalar_type() == at::kFloat8_e8m0fnu ||
         t.scalar_type() == at::kFloat8_e4m3fn;
}

// ------------------------------------------------------------- tiled weights

// The identity of a tensor's contents: its storage (held weakly, so a freed weight
// whose address is reused is not mistaken for the old one), address and version.
struct TensorStamp {
  std::optional<c10::weak_intrusive_ptr<c10::StorageImpl>> storage;
  const void* ptr = nullptr;
  int64_t version = -1;

  TensorStamp() = default;
  explicit TensorStamp(const at::Tensor& t)
      : storage(t.storage().getWeakStorageImpl()), ptr(t.data_ptr()), version(t._version()) {}
  bool same(const at::Tensor& t) const {
    if (!storage || storage->expired() || ptr != t.data_ptr() || version != t._version()) return false;
    return storage->lock().get() == t.storage().unsafeGetStorageImpl();
  }
  bool expired() const { return !storage || storage->expired(); }
};

struct Tiled {
  TensorStamp w, s;
  at::Tensor tiled, tiled_s;  // tiled_s: MX scales, or the 128-row block-FP8 scales
};

std::mutex g_mu;
// (device, weight ptr, scale ptr, fmt, N, K, kind) -> tiled copy
using TileKey = std::tuple<int, const void*, const void*, int, int64_t, int64_t, int>;
std::map<TileKey, Tiled> g_tiles;
TileKey g_sweep_at{};  // where the bounded sweep resumes

// Drop cached copies whose weight or scale storage has been freed: `budget` entries
// from where the last sweep stopped (all of them for budget < 0).  Caller holds g_mu.
void sweep_tiles(int budget) {
  if (g_tiles.empty()) return;
  const size_t n = budget < 0 ? g_tiles.size() : std::min<size_t>((size_t)budget, g_tiles.size());
  auto it = g_tiles.lower_bound(g_sweep_at);
  for (size_t i = 0; i < n; ++i) {
    if (it == g_tiles.end()) it = g_tiles.begin();
    if (it->second.w.expired() || it->second.s.expired()) it = g_tiles.erase(it);
    else ++it;
    if (g_tiles.empty()) return;
  }
  g_sweep_at = it == g_tiles.end() ? TileKey{} : it->first;
}

constexpr int kSweepPerCall = 4;

// MX weight: codes (E4M3 [N, K] or packed FP6 [N, 3K/4]) + E8M0 scales in `scale_layout`.
// Returned by value (the tensors are reference-counted), so a concurrent re-tile of the
// same key cannot change them under the caller.
Tiled tiled_mx(const at::Tensor& w, const at::Tensor& ws, int fmt, int64_t N, int64_t K, int scale_layout,
               hipStream_t s) {
  TORCH_CHECK(w.is_cuda() && ws.is_cuda() && w.device() == ws.device(), "weights must be on one HIP device");
  TORCH_CHECK(w.is_contiguous() && ws.is_contiguous(), "weight codes and scales must be contiguous");
  const int64_t need_s = scale_layout ? mxl_swizzled_scale_bytes(N, K) : N * (K / 32);
  TORCH_CHECK(ws.numel() * ws.element_size() >= need_s, "weight scales hold ", ws.numel() * ws.element_size(),
              " bytes, need ", need_s);
  std::lock_guard<std::mutex> lock(g_mu);
  const TileKey key{(int)w.device().index(), w.data_ptr(), ws.data_ptr(), fmt, N, K, scale_layout};
  auto it = g_tiles.find(key);
  if (it != g_tiles.end() && it->second.w.same(w) && it->second.s.same(ws)) {
    Tiled hit = it->second;
    sweep_tiles(kSweepPerCall);
    return hit;
  }
  TORCH_CHECK(!capturing(s), "mach_amd: weight [", N, ", ", K, "] was not prepared before graph capture; "
              "run the shape once outside capture (warmup)");
  sweep_tiles(-1);
  Tiled t;
  auto opts = w.options().dtype(at::kByte);
  t.tiled = at::empty({mxl_tiled_weight_bytes(N, K, fmt)}, opts);
  t.tiled_s = at::empty({mxl_tiled_scale_bytes(N, K)}, opts);
  check(mxl_pack_weight_ex(w.data_ptr(), ws.data_ptr(), scale_layout, N, K, fmt, t.tiled.data_ptr(),
                           t.tiled_s.data_ptr(), s),
        "mxl_pack_weight_ex");
  t.w = TensorStamp(w);
  t.s = TensorStamp(ws);
  return g_tiles[key] = std::move(t);
}

// Block-FP8 weight: E4M3 [N, K] + the reference's 64-row duplicated scales
// sb64 [N/64, K/128] (scale.repeat_interleave(2, dim=0), fp8/linear.py:137-154),
// reduced to the 128-row block scales [ceil(N/128), K/128] this library reads.
Tiled tiled_block(const at::Tensor& w, const at::Tensor& sb64, int64_t N, int64_t K, hipStream_t s) {
  std::lock_guard<std::mutex> lock(g_mu);
  const TileKey key{(int)w.device().index(), w.data_ptr(), sb64.data_ptr(), kE4M3, N, K, 2};
  auto it = g_tiles.find(key);
  if (it != g_tiles.end() && it->second.w.same(w) && it->second.s.same(sb64)) {
    Tiled hit = it->second;
    sweep_tiles(kSweepPerCall);
    return hit;
  }
  TORCH_CHECK(!capturing(s), "mach_amd: block-FP8 weight [", N, ", ", K, "] was not prepared before graph "
              "capture; run the shape once outside capture (warmup)");
  sweep_tiles(-1);
  Tiled t;
  t.tiled = at::empty({mxl_tiled_weight_bytes(N, K, kE4M3)}, w.options().dtype(at::kByte));
  check(mxl_pack_weight(w.data_ptr(), nullptr, N, K, kE4M3, t.tiled.data_ptr(), nullptr, s), "mxl_pack_weight");
  t.tiled_s = sb64.index({at::indexing::Slice(0, at::indexing::None, 2)}).contiguous();
  t.w = TensorStamp(w);
  t.s = TensorStamp(sb64);
  return g_tiles[key] = std::move(t);
}

// --------------------------------------------------------------- workspaces

// Split-K scratch per (device, stream), grown outside capture; a superseded buffer is
// kept (a captured graph may hold its address), so none is ever freed.  A capture that
// would need a bigger buffer than its stream holds raises, as the reference's
// capture_cache_miss does (native_backend.py:163-170): running it with less scratch
// would change the K split and so the summation order of the captured result.
std::map<std::pair<int, hipStream_t>, std::vector<at::Tensor>> g_ws;

std::pair<void*, int64_t> workspace(const at::Tensor& like, int64_t nbytes, hipStream_t s) {
  if (nbytes <= 0) return {nullptr, 0};
  std::lock_guard<std::mutex> lock(g_mu);
  auto& v = g_ws[{(int)like.device().index(), s}];
  if (v.empty() || v.back().numel() < nbytes) {
    TORCH_CHECK(!capturing(s), "mach_amd: this shape needs a ", nbytes, "-byte split-K workspace but the capture "
                "stream holds ", v.empty() ? 0 : v.back().numel(), " bytes; warm this shape before capture "
                "(run it once on the capture stream outside capture)");
    const int64_t size = std::max<int64_t>(nbytes, v.empty() ? 0 : 2 * v.back().numel());
    v.push_back(at::empty({size}, like.options().dtype(at::kByte)));
  }
  return {v.back().data_ptr(), v.back().numel()};
}

mxl_gemm_options options(int sa_layout, int64_t tactic, int64_t splits) {
  mxl_gemm_options o{sa_layout, -1, 0, 0, 0, 0, 0, 0, 1.0f};
  if (tactic >= 0) {  // an explicit kernel, with the caller's split count
    o.kernel = (int)tactic;
    o.splits = splits > 0 ? (int)splits : 0;
  }
  return o;
}

// The output format and scale of the mxfp6 ops (`alpha`, `dtype`): the GEMMs scale the
// fp32 sum and round it once to bf16 or fp16.
mxl_gemm_options with_output(mxl_gemm_options o, double alpha, at::ScalarType dtype, const char* who) {
  TORCH_CHECK(dtype == at::kBFloat16 || dtype == at::kHalf, who, ": output dtype must be bfloat16 or float16, got ",
              dtype);
  TORCH_CHECK(std::isfinite(alpha) && alpha != 0.0, who, ": alpha must be finite and non-zero");
  o.out_dtype = dtype == at::kHalf ? 1 : 0;
  o.alpha = (float)alpha;
  return o;
}

at::ScalarType out_dtype_of(const mxl_gemm_options& o) { return o.out_dtype == 1 ? at::kHalf : at::kBFloat16; }

void check_act(const at::Tensor& a, int64_t K, const char* who) {
  TORCH_CHECK(a.is_cuda() && a.dim() == 2 && a.is_contiguous() && a.size(1) == K, who,
              ": activations must be a contiguous HIP tensor [M, K] with K = ", K);
}

// MX GEMM on MXFP8 activations a [M, K] (scales in sa_layout) and a tiled weight.
at::Tensor mx_gemm(const at::Tensor& a, const at::Tensor& sa, int sa_layout, const Tiled& t, int fmt, int64_t N,
                   int64_t K, const mxl_gemm_options& o, const at::Tensor& out_opt, const at::Tensor& ws_opt,
                   hipStream_t s) {
  const int64_t M = a.size(0);
  at::Tensor out = out_opt.defined() ? out_opt : at::empty({M, N}, a.options().dtype(out_dtype_of(o)));
  TORCH_CHECK(out.scalar_type() == out_dtype_of(o) && out.dim() == 2 && out.size(0) == M && out.size(1) == N &&
                  out.stride(1) == 1 && out.stride(0) >= N,
              "out must be ", out_dtype_of(o), " [M, N] with unit column stride");
  const int64_t need_s = sa_layout ? mxl_swizzled_scale_bytes(M, K) : M * (K / 32);
  TORCH_CHECK(sa.is_cuda() && sa.is_contiguous() && sa.numel() * sa.element_size() >= need_s,
              "activation scales hold ", sa.numel() * sa.element_size(), " bytes, need ", need_s);
  if (M == 0) return out;
  const int64_t nbytes = mxl_gemm_workspace_bytes_ex(M, N, K, fmt, 0, &o);
  std::pair<void*, int64_t> w;
  if (ws_opt.defined() && ws_opt.numel() >= nbytes) w = {ws_opt.data_ptr(), ws_opt.numel()};
  else w = workspace(a, nbytes, s);
  check(mxl_mx_gemm_ex(a.data_ptr(), sa.data_ptr(), M, t.tiled.data_ptr(), t.tiled_s.data_ptr(), N, K, fmt, nullptr,
                       out.data_ptr(), out.stride(0), w.first, w.second, &o, s),
        "mxl_mx_gemm_ex");
  return out;
}

std::tuple<at::Tensor, at::Tensor> quantize_logical(const at::Tensor& x, int rule, hipStream_t s) {
  TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kBFloat16 && x.dim() == 2 && x.size(1) % 32 == 0,
              "quantize_mxfp8 needs a bf16 HIP tensor [M, K] with K % 32 == 0");
  at::Tensor xc = x.stride(1) == 1 ? x : x.contiguous();
  const int64_t M = xc.size(0), K = xc.size(1);
  at::Tensor codes = at::empty({M, K}, xc.options().dtype(at::kFloat8_e4m3fn));
  at::Tensor scales = at::empty({M, K / 32}, xc.options().dtype(at::kByte));
  if (M) check(mxl_quantize_mxfp8(xc.data_ptr(), M, K, xc.stride(0), rule, codes.data_ptr(), scales.data_ptr(), s),
               "mxl_quantize_mxfp8");
  return {codes, scales};
}

// Up to 16 bf16 rows quantized inside the weight-streaming GEMM's own wavefronts (one
// launch, the same bits as quantize + GEMM); nullopt for shapes that take the two calls
// (the one-launch handoff measured slower than the two launches).
std::optional<at::Tensor> quant_row(const at::Tensor& x, const Tiled& t, int fmt, int64_t N, int64_t K,
                                    const mxl_gemm_options& o, hipStream_t s) {
  const int64_t M = x.size(0);
  if (M < 1 || M > 16 || !mxl_producer_gemm_supported(3, M, K, kFloorCarry175, fmt) ||
      x.scalar_type() != at::kBFloat16 || !x.is_cuda())
    return {};
  at::Tensor xc = x.contiguous();
  at::Tensor out = at::empty({M, N}, xc.options().dtype(out_dtype_of(o)));
  check(mxl_quant_mx_gemm_ex(xc.data_ptr(), M, K, kFloorCarry175, t.tiled.data_ptr(), t.tiled_s.data_ptr(), N, fmt,
                             nullptr, out.data_ptr(), N, &o, s),
        "mxl_quant_mx_gemm_ex");
  return out;
}

// ================================================== vllm_mach_block_fp8::mm

// a E4M3 [M, K]; b = weight.T (E4M3 [K, N], stride (1, K)); sa fp32 [M, K/128],
// stride (1, M); sb = sb64.T (fp32 [K/128, N/64], stride (1, K/128)).  bf16 [M, N].
at::Tensor block_fp8_mm(const at::Tensor& a, const at::Tensor& b, const at::Tensor& sa, const at::Tensor& sb) {
  TORCH_CHECK(a.is_cuda() && a.dim() == 2 && a.is_contiguous() && a.scalar_type() == at::kFloat8_e4m3fn,
              "vllm_mach_block_fp8::mm: a must be contiguous E4M3 [M, K]");
  const int64_t M = a.size(0), K = a.size(1);
  TORCH_CHECK(b.scalar_type() == at::kFloat8_e4m3fn && b.dim() == 2 && b.size(0) == K && b.stride(0) == 1 &&
                  b.stride(1) == K,
              "vllm_mach_block_fp8::mm: b must be the transposed view [K, N] of an E4M3 weight [N, K]");
  const int64_t N = b.size(1);
  TORCH_CHECK(K % 128 == 0 && N % 64 == 0, "vllm_mach_block_fp8::mm: need K % 128 == 0 and N % 64 == 0");
  TORCH_CHECK(sa.scalar_type() == at::kFloat && sa.dim() == 2 && sa.size(0) == M && sa.size(1) == K / 128 &&
                  (M <= 1 || (sa.stride(0) == 1 && sa.stride(1) == M)) && (M != 1 || K == 128 || sa.stride(1) == 1),
              "vllm_mach_block_fp8::mm: sa must be fp32 [M, K/128] with stride (1, M)");
  TORCH_CHECK(sb.scalar_type() == at::kFloat && sb.dim() == 2 && sb.size(0) == K / 128 && sb.size(1) == N / 64 &&
                  sb.stride(0) == 1 && sb.stride(1) == K / 128,
              "vllm_mach_block_fp8::mm: sb must be the transposed view [K/128, N/64] of the 64-row scales");
  TORCH_CHECK(b.device() == a.device() && sa.device() == a.device() && sb.device() == a.device(),
              "vllm_mach_block_fp8::mm: operands on different devices");
  hipStream_t s = stream_of(a);
  const Tiled t = tiled_block(b.t(), sb.t(), N, K, s);
  at::Tensor out = at::empty({M, N}, a.options().dtype(at::kBFloat16));
  if (M == 0) return out;
  const mxl_gemm_options o = options(0, -1, 0);
  auto w = workspace(a, mxl_gemm_workspace_bytes_ex(M, N, K, kE4M3, 1, &o), s);
  check(mxl_block_fp8_gemm_ex(a.data_ptr(), sa.data_ptr(), M, t.tiled.data_ptr(), t.tiled_s.data_ptr(), N, K, nullptr,
                              out.data_ptr(), N, w.first, w.second, &o, s),
        "mxl_block_fp8_gemm_ex");
  return out;
}

// ================================================ mach_fp8_activation::run

void fp8_activation_run(at::Tensor& out, const at::Tensor& input, at::Tensor& scales, bool is_scale_transposed) {
  TORCH_CHECK(input.is_cuda() && input.scalar_type() == at::kBFloat16 && input.dim() == 2 && input.is_contiguous(),
              "mach_fp8_activation::run: input must be contiguous bf16 [rows, 2H]");
  const int64_t rows = input.size(0), H = input.size(1) / 2;
  TORCH_CHECK(input.size(1) % 256 == 0, "mach_fp8_activation::run: H must be a multiple of 128");
  TORCH_CHECK(out.scalar_type() == at::kFloat8_e4m3fn && out.dim() == 2 && out.size(0) == rows && out.size(1) == H &&
                  out.is_contiguous(),
              "mach_fp8_activation::run: out must be contiguous E4M3 [rows, H]");
  TORCH_CHECK(scales.scalar_type() == at::kFloat && scales.dim() == 2 && scales.size(0) == rows &&
                  scales.size(1) == H / 128,
              "mach_fp8_activation::run: scales must be fp32 [rows, H/128]");
  if (is_scale_transposed) {
    TORCH_CHECK((rows <= 1 || (scales.stride(0) == 1 && scales.stride(1) == rows)) &&
                    (rows != 1 || H == 128 || scales.stride(1) == 1),
                "mach_fp8_activation::run: transposed scales need stride (1, rows)");
  } else {
    TORCH_CHECK(scales.is_contiguous(), "mach_fp8_activation::run: scales must be contiguous");
  }
  TORCH_CHECK(out.device() == input.device() && scales.device() == input.device(),
              "mach_fp8_activation::run: operands on different devices");
  if (rows == 0) return;
  check(mxl_silu_mul_block_fp8(input.data_ptr(), rows, H, is_scale_transposed ? 1 : 0, out.data_ptr(),
                               scales.data_ptr(), stream_of(input)),
        "mxl_silu_mul_block_fp8");
}

// ============================================================ mxfp8_sm120

// The reference's native MXFP8 GEMM: a E4M3 [M, K], b E4M3 [N, K], sa and sb the
// swizzled E8M0 scales of a and b.  tactic -1 lets the cost model choose (splits,
// swizzle and sms are then unused); tactic k >= 0 forces kernel k with `splits` K
// splits.  swizzle, sms and use_pdl tune the reference's CUTLASS launch and have
// no counterpart here (HIP graphs overlap the launches).
at::Tensor mxfp8_gemm(const at::Tensor& a, const at::Tensor& b, const at::Tensor& sa, const at::Tensor& sb,
                      const c10::optional<at::Tensor>& out, const c10::optional<at::Tensor>& ws, int64_t tactic,
                      int64_t splits, int64_t swizzle, int64_t sms, bool use_pdl) {
  (void)swizzle; (void)sms; (void)use_pdl;
  TORCH_CHECK(is_byte_dtype(a) && a.element_size() == 1, "mxfp8_sm120::gemm: a must hold E4M3 codes");
  TORCH_CHECK(b.dim() == 2 && b.scalar_type() == at::kFloat8_e4m3fn, "mxfp8_sm120::gemm: b must be E4M3 [N, K]");
  const int64_t N = b.size(0), K = b.size(1);
  check_act(a, K, "mxfp8_sm120::gemm");
  TORCH_CHECK(N % 16 == 0 && K % 128 == 0, "mxfp8_sm120::gemm: need N % 16 == 0 and K % 128 == 0");
  hipStream_t s = stream_of(a);
  const Tiled t = tiled_mx(b, sb, kE4M3, N, K, 1, s);
  return mx_gemm(a, sa, 1, t, kE4M3, N, K, options(1, tactic, splits), out.value_or(at::Tensor()),
                 ws.value_or(at::Tensor()), s);
}

// Prepares the weight's tiled copy and returns the split-K workspace the same call
// to gemm would use (an empty tensor when it needs none).
at::Tensor mxfp8_allocate_workspace(const at::Tensor& a, const at::Tensor& b, const at::Tensor& sa,
                                    const at::Tensor& sb, const at::Tensor& out, int64_t tactic, int64_t splits,
                                    int64_t swizzle, int64_t sms) {
  (void)sa; (void)out; (void)swizzle; (void)sms;
  TORCH_CHECK(b.dim() == 2 && b.scalar_type() == at::kFloat8_e4m3fn, "mxfp8_sm120::allocate_workspace: b must be "
              "E4M3 [N, K]");
  const int64_t N = b.size(0), K = b.size(1);
  hipStream_t s = stream_of(b);
  tiled_mx(b, sb, kE4M3, N, K, 1, s);
  const mxl_gemm_options o = options(1, tactic, splits);
  return at::empty({mxl_gemm_workspace_bytes_ex(a.size(0), N, K, kE4M3, 0, &o)}, b.options().dtype(at::kByte));
}

// x bf16 [M, K] quantized on the fly (floor_carry175), w E4M3 [N, K], ws swizzled scales.
at::Tensor mxfp8_gemm_from_float(const at::Tensor& x, const at::Tensor& w, const at::Tensor& ws) {
  TORCH_CHECK(w.dim() == 2 && w.scalar_type() == at::kFloat8_e4m3fn, "mxfp8_sm120::gemm_from_float: w must be E4M3 "
              "[N, K]");
  const int64_t N = w.size(0), K = w.size(1);
  TORCH_CHECK(x.dim() == 2 && x.size(1) == K, "mxfp8_sm120::gemm_from_float: x must be [M, K]");
  hipStream_t s = stream_of(x);
  const Tiled t = tiled_mx(w, ws, kE4M3, N, K, 1, s);
  if (auto y = quant_row(x, t, kE4M3, N, K, options(0, -1, 0), s)) return *y;
  auto q = quantize_logical(x, kFloorCarry175, s);
  return mx_gemm(std::get<0>(q), std::get<1>(q), 0, t, kE4M3, N, K, options(0, -1, 0), at::Tensor(), at::Tensor(), s);
}

// Two-limb MXFP8 GEMM (M <= 64): out = bf16(hi . W^T + res . W^T), the limbs' fp32
// products summed before the one rounding.  hi / res E4M3 [M, K] with swizzled scales
// s_hi / s_res; weight E4M3 [N, K] with swizzled s_weight (flat, as the reference
// passes scale.view(-1)).
void mxfp8_dual_gemm_out(const at::Tensor& hi, const at::Tensor& weight, const at::Tensor& s_hi,
                         const at::Tensor& s_weight, const at::Tensor& res, const at::Tensor& s_res, at::Tensor& out) {
  TORCH_CHECK(weight.dim() == 2 && weight.scalar_type() == at::kFloat8_e4m3fn,
              "mxfp8_sm120::dual_gemm_out: weight must be E4M3 [N, K]");
  const int64_t N = weight.size(0), K = weight.size(1);
  TORCH_CHECK(is_byte_dtype(hi) && hi.element_size() == 1 && is_byte_dtype(res) && res.element_size() == 1,
              "mxfp8_sm120::dual_gemm_out: hi and res must hold E4M3 codes");
  check_act(hi, K, "mxfp8_sm120::dual_gemm_out");
  check_act(res, K, "mxfp8_sm120::dual_gemm_out");
  const int64_t M = hi.size(0);
  TORCH_CHECK(res.size(0) == M && M <= 64, "mxfp8_sm120::dual_gemm_out: hi and res must be [M, K] with M <= 64");
  TORCH_CHECK(N % 16 == 0 && K % 128 == 0, "mxfp8_sm120::dual_gemm_out: need N % 16 == 0 and K % 128 == 0");
  TORCH_CHECK(out.scalar_type() == at::kBFloat16 && out.dim() == 2 && out.size(0) == M && out.size(1) == N &&
                  out.stride(1) == 1 && out.stride(0) >= N,
              "mxfp8_sm120::dual_gemm_out: out must be bf16 [M, N] with unit column stride");
  const int64_t need_s = mxl_swizzled_scale_bytes(M, K);
  for (const at::Tensor* t : {&s_hi, &s_res})
    TORCH_CHECK(t->is_cuda() && t->is_contiguous() && t->numel() * t->element_size() >= need_s,
                "mxfp8_sm120::dual_gemm_out: activation scales hold ", t->numel() * t->element_size(),
                " bytes, need ", need_s);
  hipStream_t s = stream_of(hi);
  const Tiled t = tiled_mx(weight, s_weight, kE4M3, N, K, 1, s);
  if (M == 0) return;
  // the two limbs' partials
  const int64_t nbytes = 2 * M * N * 4;
  auto w = workspace(hi, nbytes, s);
  const mxl_gemm_options o = options(1, -1, 0);
  check(mxl_mx_gemm_dual_ex(hi.data_ptr(), s_hi.data_ptr(), res.data_ptr(), s_res.data_ptr(), M, t.tiled.data_ptr(),
                            t.tiled_s.data_ptr(), N, K, kE4M3, nullptr, out.data_ptr(), out.stride(0), w.first,
                            w.second, &o, s),
        "mxl_mx_gemm_dual_ex");
}

// ================================================================== mxfp6

std::tuple<at::Tensor, at::Tensor> mxfp6_quantize_mxfp8(const at::Tensor& x) {
  TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kBFloat16 && x.dim() == 2 && x.size(1) % 32 == 0,
              "mxfp6::quantize_mxfp8 needs a bf16 HIP tensor [M, K] with K % 32 == 0");
  at::Tensor xc = x.stride(1) == 1 ? x : x.contiguous();
  const int64_t M = xc.size(0), K = xc.size(1);
  at::Tensor codes = at::empty({M, K}, xc.options().dtype(at::kByte));
  at::Tensor scales = at::empty({mxl_swizzled_scale_bytes(M, K)}, xc.options().dtype(at::kByte));
  if (M)
    check(mxl_quantize_mxfp8_swizzled(xc.data_ptr(), M, K, xc.stride(0), kFloorCarry175, codes.data_ptr(),
                                      scales.data_ptr(), stream_of(xc)),
          "mxl_quantize_mxfp8_swizzled");
  return {codes, scales};
}

std::tuple<at::Tensor, at::Tensor> mxfp6_quantize_mxfp8_logical(const at::Tensor& x) {
  return quantize_logical(x, kFloorCarry175, stream_of(x));
}

// logical E8M0 [R, K/32] (or [E, R, K/32]: each expert swizzled on its own) -> swizzled.
at::Tensor mxfp6_pack_scales(const at::Tensor& scales) {
  TORCH_CHECK(scales.is_cuda() && is_byte_dtype(scales) && (scales.dim() == 2 || scales.dim() == 3),
              "mxfp6::pack_scales needs E8M0 bytes [R, K/32] or [E, R, K/32] on a HIP device");
  at::Tensor sc = scales.contiguous();
  const int64_t E = sc.dim() == 3 ? sc.size(0) : 1;
  const int64_t R = sc.size(sc.dim() - 2), K = sc.size(sc.dim() - 1) * 32;
  const int64_t per = mxl_swizzled_scale_bytes(R, K);
  at::Tensor out = at::empty(sc.dim() == 3 ? std::vector<int64_t>{E, per} : std::vector<int64_t>{per},
                             sc.options().dtype(at::kByte));
  hipStream_t s = stream_of(sc);
  const uint8_t* src = static_cast<const uint8_t*>(sc.data_ptr());
  uint8_t* dst = static_cast<uint8_t*>(out.data_ptr());
  for (int64_t e = 0; e < E; ++e)
    check(mxl_swizzle_scales(src + e * R * (K / 32), R, K, dst + e * per, s), "mxl_swizzle_scales");
  return out;
}

// W6A8: x bf16 [M, K] quantized on the fly, w packed FP6 E3M2 [N, 3K/4], ws swizzled.
at::Tensor mxfp6_gemm_from_float(const at::Tensor& x, const at::Tensor& w, const at::Tensor& ws, int64_t N,
                                 double alpha, at::ScalarType dtype) {
  TORCH_CHECK(w.dim() == 2 && w.scalar_type() == at::kByte && w.size(0) == N && w.size(1) % 3 == 0,
              "mxfp6::gemm_from_float: w must be packed FP6 bytes [N, 3K/4]");
  const int64_t K = w.size(1) * 4 / 3;
  TORCH_CHECK(x.dim() == 2 && x.size(1) == K && K % 128 == 0, "mxfp6::gemm_from_float: x must be [M, K], K % 128 == 0");
  hipStream_t s = stream_of(x);
  const Tiled t = tiled_mx(w, ws, kE3M2, N, K, 1, s);
  const mxl_gemm_options o = with_output(options(0, -1, 0), alpha, dtype, "mxfp6::gemm_from_float");
  if (auto y = quant_row(x, t, kE3M2, N, K, o, s)) return *y;
  auto q = quantize_logical(x, kFloorCarry175, s);
  return mx_gemm(std::get<0>(q), std::get<1>(q), 0, t, kE3M2, N, K, o, at::Tensor(), at::Tensor(), s);
}

// SwiGLU (ceil_div448 with the bf16 SiLU rounding) -> MXFP8 -> W6A8 down projection;
// one launch for one row.
at::Tensor mxfp6_gemm_from_swiglu(const at::Tensor& gate_up, const at::Tensor& w, const at::Tensor& ws, int64_t N,
                                  double alpha, at::ScalarType dtype) {
  TORCH_CHECK(gate_up.is_cuda() && gate_up.scalar_type() == at::kBFloat16 && gate_up.dim() == 2 &&
                  gate_up.is_contiguous(),
              "mxfp6::gemm_from_swiglu: gate_up must be contiguous bf16 [M, 2K]");
  TORCH_CHECK(w.dim() == 2 && w.scalar_type() == at::kByte && w.size(0) == N && w.size(1) % 3 == 0,
              "mxfp6::gemm_from_swiglu: w must be packed FP6 bytes [N, 3K/4]");
  const int64_t K = w.size(1) * 4 / 3, M = gate_up.size(0);
  TORCH_CHECK(gate_up.size(1) == 2 * K && K % 128 == 0, "mxfp6::gemm_from_swiglu: gate_up width must be 2K");
  hipStream_t s = stream_of(gate_up);
  const Tiled t = tiled_mx(w, ws, kE3M2, N, K, 1, s);
  const mxl_gemm_options o = with_output(options(0, -1, 0), alpha, dtype, "mxfp6::gemm_from_swiglu");
  at::Tensor out = at::empty({M, N}, gate_up.options().dtype(out_dtype_of(o)));
  if (M == 0) return out;
  if (M == 1 && mxl_producer_gemm_supported(0, M, K, kCeilDiv448, kE3M2)) {
    check(mxl_swiglu_mx_gemm_ex(gate_up.data_ptr(), M, K, kCeilDiv448, t.tiled.data_ptr(), t.tiled_s.data_ptr(), N,
                                kE3M2, nullptr, out.data_ptr(), N, &o, s),
          "mxl_swiglu_mx_gemm_ex");
    return out;
  }
  at::Tensor codes = at::empty({M, K}, gate_up.options().dtype(at::kByte));
  at::Tensor scales = at::empty({M, K / 32}, gate_up.options().dtype(at::kByte));
  check(mxl_swiglu_mxfp8(gate_up.data_ptr(), M, K, kCeilDiv448, 0, codes.data_ptr(), scales.data_ptr(), s),
        "mxl_swiglu_mxfp8");
  return mx_gemm(codes, scales, 0, t, kE3M2, N, K, o, out, at::Tensor(), s);
}

// Pre-quantized W6A8: codes [M, K] with swizzled activation scales.
at::Tensor mxfp6_gemm_w6a8(const at::Tensor& codes, const at::Tensor& w, const at::Tensor& scales,
                           const at::Tensor& ws, int64_t M, int64_t N, int64_t K, double alpha, at::ScalarType dtype) {
  TORCH_CHECK(is_byte_dtype(codes) && codes.element_size() == 1 && codes.dim() == 2 && codes.size(0) == M,
              "mxfp6::gemm_w6a8_pdl: codes must be E4M3 bytes [M, K]");
  TORCH_CHECK(w.dim() == 2 && w.scalar_type() == at::kByte && w.size(0) == N && w.size(1) * 4 == 3 * K,
              "mxfp6::gemm_w6a8_pdl: w must be packed FP6 bytes [N, 3K/4]");
  check_act(codes, K, "mxfp6::gemm_w6a8_pdl");
  hipStream_t s = stream_of(codes);
  const Tiled t = tiled_mx(w, ws, kE3M2, N, K, 1, s);
  return mx_gemm(codes, scales, 1, t, kE3M2, N, K, with_output(options(1, -1, 0), alpha, dtype, "mxfp6::gemm_w6a8_pdl"),
                 at::Tensor(), at::Tensor(), s);
}

}  // namespace

TORCH_LIBRARY(vllm_mach_block_fp8, m) { m.def("mm(Tensor a, Tensor b, Tensor sa, Tensor sb) -> Tensor"); }
TORCH_LIBRARY_IMPL(vllm_mach_block_fp8, CUDA, m) { m.impl("mm", &block_fp8_mm); }

TORCH_LIBRARY(mach_fp8_activation, m) {
  m.def("run(Tensor(a!) out, Tensor input, Tensor(b!) scales, bool is_scale_transposed) -> ()");
}
TORCH_LIBRARY_IMPL(mach_fp8_activation, CUDA, m) { m.impl("run", &fp8_activation_run); }

TORCH_LIBRARY(mxfp8_sm120, m) {
  m.def("gemm(Tensor a, Tensor b, Tensor sa, Tensor sb, Tensor(a!)? out=None, Tensor? workspace=None, "
        "int tactic=-1, int splits=1, int swizzle=1, int sms=0, bool use_pdl=False) -> Tensor");
  m.def("allocate_workspace(Tensor a, Tensor b, Tensor sa, Tensor sb, Tensor out, int tactic, int splits, "
        "int swizzle, int sms) -> Tensor");
  m.def("gemm_from_float(Tensor x, Tensor w, Tensor ws) -> Tensor");
  // the programmatic-dependent-launch entry points of the reference's PDL build
  // (dense_mxfp8.py:54-70): the same work here, where a HIP graph carries the overlap
  m.def("gemm_pdl(Tensor a, Tensor b, Tensor sa, Tensor sb, Tensor(a!)? out=None, Tensor? workspace=None, "
        "int tactic=-1, int splits=1, int swizzle=1, int sms=0, bool use_pdl=False) -> Tensor");
  m.def("gemm_from_float_pdl(Tensor x, Tensor w, Tensor ws) -> Tensor");
  m.def("dual_gemm_out(Tensor hi, Tensor weight, Tensor s_hi, Tensor s_weight, Tensor res, Tensor s_res, "
        "Tensor(a!) out) -> ()");
}
TORCH_LIBRARY_IMPL(mxfp8_sm120, CUDA, m) {
  m.impl("gemm", &mxfp8_gemm);
  m.impl("allocate_workspace", &mxfp8_allocate_workspace);
  m.impl("gemm_from_float", &mxfp8_gemm_from_float);
  m.impl("gemm_pdl", &mxfp8_gemm);
  m.impl("gemm_from_float_pdl", &mxfp8_gemm_from_float);
  m.impl("dual_gemm_out", &mxfp8_dual_gemm_out);
}

TORCH_LIBRARY(mxfp6, m) {
  m.def("quantize_mxfp8(Tensor x) -> (Tensor, Tensor)");
  m.def("quantize_mxfp8_logical(Tensor x) -> (Tensor, Tensor)");
  m.def("quantize_mxfp8_pdl(Tensor x) -> (Tensor, Tensor)");
  m.def("pack_scales(Tensor scales) -> Tensor");
  m.def("gemm_from_float(Tensor x, Tensor w, Tensor ws, int N, float alpha, ScalarType dtype) -> Tensor");
  m.def("gemm_from_swiglu(Tensor gate_up, Tensor w, Tensor ws, int N, float alpha, ScalarType dtype) -> Tensor");
  m.def("gemm_w6a8_pdl(Tensor codes, Tensor w, Tensor scales, Tensor ws, int M, int N, int K, float alpha, "
        "ScalarType dtype) -> Tensor");
}
TORCH_LIBRARY_IMPL(mxfp6, CUDA, m) {
  m.impl("quantize_mxfp8", &mxfp6_quantize_mxfp8);
  m.impl("quantize_mxfp8_logical", &mxfp6_quantize_mxfp8_logical);
  m.impl("quantize_mxfp8_pdl", &mxfp6_quantize_mxfp8);
  m.impl("pack_scales", &mxfp6_pack_scales);
  m.impl("gemm_from_float", &mxfp6_gemm_from_float);
  m.impl("gemm_from_swiglu", &mxfp6_gemm_from_swiglu);
  m.impl("gemm_w6a8_pdl", &mxfp6_gemm_w6a8);
}
