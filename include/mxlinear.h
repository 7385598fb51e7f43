/*
 * mxlinear.h -- C ABI of the MI355X (gfx950) quantized-linear library
 * (libmxlinear.so).  Plain pointers and sizes; every device pointer is HIP
 * device memory and every call enqueues on `stream` (a hipStream_t, may be 0).
 *
 * Status-returning entry points return 0 on success and a negative code on
 * failure (MXL_EINVAL -1: bad argument, nothing launched; MXL_EHIP -2: a HIP
 * launch failed); mxl_last_error() then describes the failure (thread-local).
 *
 * Formats:  fmt 0 = E4M3 (8-bit codes), 2 = E2M3, 3 = E3M2 (FP6 packed four
 * values per three bytes, little-endian 6-bit fields: value i of a group in
 * bits [6i, 6i+6)).  Scales are E8M0 bytes (2^(s-127)), one per 32 along K.
 * rule 0 = floor_carry175 (the reference quantizer quantize_block,
 * src/vllm_mach/mxfp8/reconstruct_model.py:34-50), rule 1 = ceil_div448
 * (src/vllm_mach/mxfp6/mxfp8_mlp.py:100-105), rule 2 = rp_ue8m0 (FlashInfer's
 * mxfp8_quantize convention as src/vllm_mach/mxfp8/swiglu_quant.py:58-66 writes
 * it: amax * (1/448) rounded up onto E8M0, saturating; codes of the clamped
 * +-448 products; quantizers, dual and SwiGLU only).
 *
 * Each declaration cites the reference interface (troycheng/vllm-mach
 * v0.4.0) it replaces.
 */
#ifndef MXLINEAR_H
#define MXLINEAR_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXL_OK 0
#define MXL_EINVAL -1
#define MXL_EHIP -2
#define MXL_EUNSUPPORTED -3

/* Library identity and error text.  Counterpart of the reference's ABI/schema
 * verification (src/vllm_mach/mxfp8/native_backend.py:76-97). */
int mxl_version(void);
const char* mxl_last_error(void);

/* 1 if `device` is gfx950, 0 if not, <0 if HIP cannot be queried.  Replaces
 * the SM120 capability gate (src/vllm_mach/mxfp6/dense.py:83-110). */
int mxl_device_supported(int device);

/* Dynamic MXFP8 activation quantization: bf16 x [M, K] (row stride ldx
 * elements) -> E4M3 codes [M, K] + E8M0 scales [M, K/32], row-major.
 * K % 32 == 0.  Replaces torch.ops.mxfp6.quantize_mxfp8 / quantize_mxfp8_logical
 * (src/vllm_mach/mxfp6/dense_mxfp8.py:40, src/vllm_mach/mxfp6/moe_utils.py:172-202). */
int mxl_quantize_mxfp8(const void* x, int64_t M, int64_t K, int64_t ldx, int rule,
                       void* codes, void* scales, void* stream);

/* The same quantization with the scales in the reference's swizzled layout
 * (128-row x 4-group tiles: byte (r, g) at (((r/128 T + g/4) 32 + r%32) 4 +
 * (r%128)/32) 4 + g%4, T = ceil(K/128), padding bytes zeroed;
 * mxl_swizzled_scale_bytes(M, K) bytes), the layout the reference's GEMMs read.
 * Replaces vLLM's mxfp8_e4m3_quantize(x, is_sf_swizzled_layout=True)
 * (src/vllm_mach/mxfp8/native_backend.py:287-293) and the packed-scale
 * torch.ops.mxfp6.quantize_mxfp8 (src/vllm_mach/mxfp6/moe_utils.py:285-317). */
int mxl_quantize_mxfp8_swizzled(const void* x, int64_t M, int64_t K, int64_t ldx, int rule, void* codes,
                                void* scales, void* stream);

/* MXFP6 weight quantization (OCP MX v1.0 floor rule): bf16 x [M, K] (row
 * stride ldx elements) -> packed FP6 [M, 3K/4] (fmt 2 = E2M3, 3 = E3M2) + E8M0
 * [M, K/32].  Replaces the offline MXFP6 quantizer the reference's checkpoints
 * and tests come from (mxfp6.quantize_mxfp6, tests/native_mxfp6/test_moe.py:179-184,
 * tests/native_mxfp6/test_mxfp6_sm120.py:37). */
int mxl_quantize_mxfp6(const void* x, int64_t M, int64_t K, int64_t ldx, int fmt, void* packed, void* scales,
                       void* stream);

/* Bytes of the swizzled scale buffer for [M, K] (mxfp8_mlp.py:122). */
int64_t mxl_swizzled_scale_bytes(int64_t M, int64_t K);

/* Logical E8M0 scales [R, K/32] -> the swizzled layout (padding zeroed).
 * Replaces pack_scales (src/vllm_mach/mxfp6/moe_utils.py:162-164,
 * src/vllm_mach/mxfp6/dense_mxfp8.py:150-151), whose output this library's
 * GEMMs read as swizzled scales. */
int mxl_swizzle_scales(const void* logical, int64_t R, int64_t K, void* swizzled, void* stream);

/* SwiGLU -> MXFP8 producer: gate_up bf16 [M, 2K] (gate = cols [0, K), up =
 * [K, 2K)) -> codes [M, K] + scales, logical [M, K/32] (swizzled = 0) or the
 * reference's swizzled layout (swizzled = 1, padding zeroed).  Rules 0 and 1
 * round the SiLU to bf16 before the product; replaces _silu_quant /
 * _triton_quantize (src/vllm_mach/mxfp6/mxfp8_mlp.py:87-127).  Rule 2 rounds
 * once, bf16((g / (1 + exp(-g))) * up); replaces the champion producer
 * swiglu_quant._kernel (src/vllm_mach/mxfp8/swiglu_quant.py:46-70). */
int mxl_swiglu_mxfp8(const void* gate_up, int64_t M, int64_t K, int rule, int swizzled,
                     void* codes, void* scales, void* stream);

/* Residual add + Gemma RMSNorm -> MXFP8 producer feeding gate_up: per row of N
 * (32 <= N <= 16384, N % 32 == 0), x' = x + residual (fp32; residual may be
 * null), summed = bf16(x') (written when residual is given), y = bf16((x' *
 * rsqrt(mean(x'^2) + eps)) * (weight + 1)), then E4M3 codes [M, N] and E8M0
 * scales of y per 32 (rule, logical [M, N/32] or swizzled as in
 * mxl_swiglu_mxfp8).  The rsqrt is 1 / sqrt with IEEE sqrt and divide.
 * Replaces _norm_quant / quantize (src/vllm_mach/mxfp6/mxfp8_norm_quant.py:15-49). */
int mxl_rmsnorm_mxfp8(const void* x, const void* residual, const void* weight, int64_t M, int64_t N, float eps,
                      int rule, int swizzled, void* codes, void* scales, void* summed, void* stream);

/* The same residual add + Gemma RMSNorm with a bf16 output y [M, N] instead of
 * MXFP8.  Replaces _norm / _impl (src/vllm_mach/mxfp6/gemma_norm.py:13-41). */
int mxl_gemma_rmsnorm(const void* x, const void* residual, const void* weight, int64_t M, int64_t N, float eps,
                      void* y, void* summed, void* stream);

/* Two-limb MXFP8 activations: per 32-block, hi = MXFP8(x) under `rule`, the
 * residual r = bf16(x - dequant(hi)), res = MXFP8(r) under the same rule; codes
 * [M, K] and logical scales [M, K/32] for each limb.  The contract of the
 * reference's dual quantizer (src/vllm_mach/mxfp8/dual.py:45-47, from the
 * absent mxfp6 wheel: this rule is this library's definition). */
int mxl_quantize_mxfp8_dual(const void* x, int64_t M, int64_t K, int64_t ldx, int rule, void* hi, void* s_hi,
                            void* res, void* s_res, void* stream);

/* Per-token group-128 FP8 quantization: bf16 x [M, K] -> E4M3 q [M, K] +
 * fp32 scales column-major s[g * M + m].  Replaces _quantize_kernel.quantize_out
 * (src/vllm_mach/fp8/_quantize_kernel.py:7-25). */
int mxl_quantize_block_fp8(const void* x, int64_t M, int64_t K, void* q, void* s_colmajor,
                           void* stream);

/* SiLU(gate)*up -> block-FP8: bf16 input [rows, 2H] -> E4M3 q [rows, H] +
 * fp32 scales [rows, H/128] (transposed = 1: s[g * rows + r]).  Replaces
 * mach_fp8_activation::run (native/fp8_activation/activation.cu:62-104). */
int mxl_silu_mul_block_fp8(const void* input, int64_t rows, int64_t H, int transposed,
                           void* q, void* scales, void* stream);

/* Sizes of the MFMA-tiled weight layout (16-row x 512-K tiles). */
int64_t mxl_tiled_weight_bytes(int64_t N, int64_t K, int fmt);
int64_t mxl_tiled_scale_bytes(int64_t N, int64_t K);

/* Load-time repack of a logical weight (E4M3 [N, K] or packed FP6 [N, 3K/4])
 * and its E8M0 scales [N, K/32] (may be NULL: block-FP8) into the tiled
 * layout.  K % 128 == 0.  Replaces pack_scales at process_weights_after_loading
 * (src/vllm_mach/mxfp6/dense_mxfp8.py:150-151, src/vllm_mach/mxfp6/dense.py:185-188,
 * src/vllm_mach/mxfp6/moe_utils.py:162-169). */
int mxl_pack_weight(const void* codes, const void* scales, int64_t N, int64_t K, int fmt,
                    void* tiled_codes, void* tiled_scales, void* stream);

/* The same repack with the E8M0 scales given in the swizzled layout
 * (scale_layout 1, as mxl_quantize_mxfp8_swizzled writes them for N rows) or
 * logical (0).  Replaces the weight-side pack_scales input of the reference's
 * MXFP8 GEMMs, whose weight scales arrive swizzled
 * (src/vllm_mach/mxfp8/native_backend.py:266-281). */
int mxl_pack_weight_ex(const void* codes, const void* scales, int scale_layout, int64_t N, int64_t K, int fmt,
                       void* tiled_codes, void* tiled_scales, void* stream);

/* Per-call GEMM options: the activation-scale layout, the tuning overrides
 * of the reference's native GEMM (tactic, splits: _DEFAULT_CONFIG,
 * src/vllm_mach/mxfp8/native_backend.py:29) and the output format and scale of
 * mxfp6::gemm_from_float / gemm_from_swiglu / gemm_w6a8_pdl (`alpha`, `dtype`,
 * src/vllm_mach/mxfp6/dense.py:122-129, src/vllm_mach/mxfp6/fused_mlp.py:16-19).
 * A NULL options pointer means {0, -1, 0, 0, 0, 0, 0, 0, 1.0f}: logical scales,
 * everything chosen by the cost model, bf16 output, no scaling.  alpha must be
 * finite and non-zero (a zero-filled struct is rejected with MXL_EINVAL). */
typedef struct mxl_gemm_options {
  int sa_layout; /* MX activation scales: 0 logical [M, K/32], 1 swizzled */
  int kernel;    /* -1 automatic; 0 weight-streaming (M <= 16), 1 wide (M >= 64,
                    K % 256 == 0), 2 generic, 4 K-chunked weight streaming (MX,
                    M <= 128: activations stationary in registers, weights through an
                    LDS ring, fp32 partials per chunk); grouped GEMMs also 3 (96-row
                    weight-streaming units).  A kernel the shape does not admit
                    returns MXL_EUNSUPPORTED. */
  int splits;    /* 0 automatic, else the K split (wide with tile_n, generic) */
  int tile_n;    /* wide: 64-column groups per workgroup tile, 1, 2 or 4; 0 automatic */
  int tile_m;    /* wide: 16-row tiles per workgroup tile, 4 or 8; 0 automatic */
  int hybrid;    /* wide, splits == 1: whole-K full rounds, the remainder split */
  int waves;     /* wide MX dense with 128-row tiles: 4 waves per workgroup (each all
                    128 rows) or 8 (two per SIMD, each 64 rows); 0 automatic */
  int out_dtype; /* output elements: 0 bf16, 1 fp16 (dense GEMMs; the grouped and
                    two-limb GEMMs write bf16 only) */
  float alpha;   /* output scale: out = round(alpha * sum) with the fp32 sum scaled
                    in fp32 and rounded once to out_dtype (a bias is added after
                    that rounding and the sum rounded again) */
} mxl_gemm_options;

/* Scratch bytes the GEMMs may use for split-K partials at (M, N, K) (the
 * largest over weight formats and block-FP8); with a smaller workspace they
 * run unsplit. */
int64_t mxl_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* Exactly the split-K bytes mxl_mx_gemm_ex (block = 0) or
 * mxl_block_fp8_gemm_ex (block = 1) uses for this shape, format and options. */
int64_t mxl_gemm_workspace_bytes_ex(int64_t M, int64_t N, int64_t K, int w_fmt, int block,
                                    const mxl_gemm_options* options);

/* Per-shape plan overrides: a measured table's entry for exactly (M, N, K, w_fmt, block)
 * on the current device.  Replaces the reference's registration of its measured
 * projection table (set_w6a8_config per row, w6a8_config_abi for the table's ABI check:
 * src/vllm_mach/mxfp6/moe_projection.py:35-105, table
 * src/vllm_mach/mxfp6/profile/qwen35_moe_projection.json).  The entry keeps the tuning
 * fields of `options` (kernel, splits, tile_n, tile_m, hybrid, waves); every dense GEMM
 * call at that shape whose own tuning fields are automatic (NULL options included) runs
 * with them, keeping its own scale layout and epilogue, and the workspace and plan-name
 * queries report that plan.  An entry whose options do not run the shape is refused
 * (MXL_EINVAL); registering a shape again replaces its entry; at most 4096 shapes.
 * Register before warmup and graph capture (a captured graph keeps the plan it was
 * captured with).  mxl_gemm_config_abi() is the version of the fields and kernel ids an
 * entry may name (a table records the value it was measured with). */
int64_t mxl_gemm_config_abi(void);
int mxl_set_gemm_config(int64_t M, int64_t N, int64_t K, int w_fmt, int block, const mxl_gemm_options* options);
int mxl_clear_gemm_configs(void);
int64_t mxl_gemm_config_count(void);

/* Two-limb MX GEMM for M <= 64: y = bf16(hi . W^T + res . W^T) with the limbs
 * accumulated separately in fp32 (each limb's partial goes to the workspace,
 * >= 2 M N 4 bytes) and summed before the one bf16 rounding; bias as in
 * mxl_mx_gemm.  Replaces gemm_out(hi, w, s_hi, ws, residual, s_res, out)
 * (src/vllm_mach/mxfp8/dual.py:45-50, docs/mxfp8-champion.md:12). */
int mxl_mx_gemm_dual(const void* hi, const void* s_hi, const void* res, const void* s_res, int64_t M,
                     const void* w_tiled, const void* sw_tiled, int64_t N, int64_t K, int w_fmt, const void* bias,
                     void* out, int64_t ldc, void* workspace, int64_t workspace_bytes, void* stream);

/* mxl_mx_gemm_dual with per-call options (NULL: the defaults); s_hi and s_res are
 * read in options->sa_layout (the other fields are unused).  Replaces
 * mxfp8_sm120::dual_gemm_out(hi, weight, s_hi, s_weight, res, s_res, out), whose
 * scales are swizzled (src/vllm_mach/mxfp8/native_backend.py:90-93). */
int mxl_mx_gemm_dual_ex(const void* hi, const void* s_hi, const void* res, const void* s_res, int64_t M,
                        const void* w_tiled, const void* sw_tiled, int64_t N, int64_t K, int w_fmt,
                        const void* bias, void* out, int64_t ldc, void* workspace, int64_t workspace_bytes,
                        const mxl_gemm_options* options, void* stream);

/* MX block-scaled GEMM: y[M, N] (bf16, row stride ldc) = A . W^T, A = E4M3
 * codes [M, K] + E8M0 [M, K/32]; W tiled (fmt 0/2/3); bias bf16 [N] or NULL
 * (added after the bf16 rounding, as y + bias in bf16).  Replaces
 * mxfp8_sm120::gemm (src/vllm_mach/mxfp6/dense_mxfp8.py:86,
 * src/vllm_mach/mxfp8/native_backend.py:77-89) and mxfp6::gemm_w6a8_pdl
 * (src/vllm_mach/mxfp6/ar_norm.py:144-147). */
int mxl_mx_gemm(const void* a, const void* sa, int64_t M, const void* w_tiled, const void* sw_tiled,
                int64_t N, int64_t K, int w_fmt, const void* bias, void* out, int64_t ldc,
                void* workspace, int64_t workspace_bytes, void* stream);

/* mxl_mx_gemm with per-call options (NULL: the defaults); sa is read in
 * options->sa_layout.  Replaces mxfp8_sm120::gemm's tactic / splits arguments
 * and its swizzled activation scales (src/vllm_mach/mxfp8/native_backend.py:77-89,
 * 193-205). */
int mxl_mx_gemm_ex(const void* a, const void* sa, int64_t M, const void* w_tiled, const void* sw_tiled, int64_t N,
                   int64_t K, int w_fmt, const void* bias, void* out, int64_t ldc, void* workspace,
                   int64_t workspace_bytes, const mxl_gemm_options* options, void* stream);

/* mxl_mx_gemm that allocates nothing: its split-K partials live in a
 * library-owned device array of mxl_noalloc_scratch_bytes() (32 MiB) per GPU,
 * so the call needs no workspace argument.  No counterpart in the reference: for
 * callers that cannot allocate (HIP graph capture, tight serving loops).  The
 * plan (kernel, tile, split) is mxl_mx_gemm's, so the result is bit-identical to
 * mxl_mx_gemm with a large enough workspace; a shape whose plan needs more
 * scratch than the array holds returns MXL_EINVAL.  `stream` must belong to the
 * current device.  All calls on one GPU share the array: calls that overlap on
 * one GPU (concurrent streams) race; every call overwrites what it reads. */
int64_t mxl_noalloc_scratch_bytes(void);
int mxl_mx_gemm_noalloc(const void* a, const void* sa, int64_t M, const void* w_tiled, const void* sw_tiled,
                        int64_t N, int64_t K, int w_fmt, const void* bias, void* out, int64_t ldc, void* stream);

/* SwiGLU -> MXFP8 -> MX GEMM for M <= 16 activation rows in one launch, bit-identical
 * to mxl_swiglu_mxfp8 (logical scales) followed by mxl_mx_gemm; rule 1 or 2, gate_up bf16
 * [M, 2K], K % 128 == 0.  M > 1: the last wavefront of every workgroup of the weight-
 * streaming GEMM is a producer wave that computes its share of the [M, K] codes with the
 * producer's arithmetic into a per-(device, stream) slot of the library's static scratch
 * (64 slots of 200 KiB per GPU, held until the process ends; a 65th stream on one device
 * returns MXL_EUNSUPPORTED), then a grid-wide handoff through device-scope counters in the
 * slot (left zero) lets the weight waves, whose weights were requested at launch, read the
 * codes.  All workgroups are resident at once (at most one per CU).  The handoff shapes:
 * K <= 7680 or 8192 < K <= 11264 (E4M3) and K <= 7680 (FP6).  M = 1: any K <= 12288, by
 * the handoff or with every wavefront recomputing the row's codes from gate_up.  Other
 * shapes return MXL_EUNSUPPORTED (use the two calls; mxl_producer_gemm_supported says which
 * run).  Calls on one stream are ordered; calls on different streams use different slots.
 * Replaces mach_swiglu_mxfp8_down at M <= 16 and mxfp6::gemm_from_swiglu's fused rows
 * (src/vllm_mach/mxfp6/mxfp8_mlp.py:15-22,71-76, src/vllm_mach/mxfp6/fused_mlp.py:13-19). */
int mxl_swiglu_mx_gemm(const void* gate_up, int64_t M, int64_t K, int rule, const void* w_tiled,
                       const void* sw_tiled, int64_t N, int w_fmt, const void* bias, void* out, int64_t ldc,
                       void* stream);

/* mxl_swiglu_mx_gemm with the output format and scale of `options` (out_dtype, alpha;
 * NULL: bf16, 1) and the scheme in options->kernel: -1 automatic (the handoff where it
 * runs), 0 the producer waves and handoff, 3 every wavefront recomputes the row (M = 1).
 * Replaces mxfp6::gemm_from_swiglu(gate_up, w, ws, N, alpha, dtype)
 * (src/vllm_mach/mxfp6/fused_mlp.py:16-19). */
int mxl_swiglu_mx_gemm_ex(const void* gate_up, int64_t M, int64_t K, int rule, const void* w_tiled,
                          const void* sw_tiled, int64_t N, int w_fmt, const void* bias, void* out, int64_t ldc,
                          const mxl_gemm_options* options, void* stream);

/* MXFP8 quantization -> MX GEMM for M <= 16 bf16 activation rows x [M, K] in one launch,
 * bit-identical to mxl_quantize_mxfp8 (rule 0, 1 or 2) followed by mxl_mx_gemm.  Two
 * schemes: the GEMM's own wavefronts quantize (M = 1: each wavefront its super-tiles' row
 * values; 2 <= M <= 16 with K <= 6144: each MFMA fragment lane the two 16-value pieces of
 * its row it multiplies, the block amax completed with the lane holding the blocks' other
 * halves; no scratch and no synchronisation beyond the workgroup), or the producer waves,
 * scratch slots, handoff and shapes of mxl_swiglu_mx_gemm.  Replaces
 * mxfp8_sm120::gemm_from_float and mxfp6::gemm_from_float at M <= 16
 * (src/vllm_mach/mxfp6/dense_mxfp8.py:89-96, src/vllm_mach/mxfp6/dense.py:122-129). */
int mxl_quant_mx_gemm(const void* x, int64_t M, int64_t K, int rule, const void* w_tiled, const void* sw_tiled,
                      int64_t N, int w_fmt, const void* bias, void* out, int64_t ldc, void* stream);

/* mxl_quant_mx_gemm with the output format, scale and scheme of `options`: -1 automatic
 * (the wavefronts' own quantization where it runs, else the handoff), 0 the producer waves
 * and handoff, 3 the wavefronts' own quantization.  Replaces mxfp6::gemm_from_float(x, w, ws, N, alpha, dtype)
 * (src/vllm_mach/mxfp6/dense.py:122-129). */
int mxl_quant_mx_gemm_ex(const void* x, int64_t M, int64_t K, int rule, const void* w_tiled, const void* sw_tiled,
                         int64_t N, int w_fmt, const void* bias, void* out, int64_t ldc,
                         const mxl_gemm_options* options, void* stream);

/* Block-FP8 activation quantization -> block-FP8 GEMM for M <= 16 bf16 rows x [M, K] in
 * one launch, bit-identical to mxl_quantize_block_fp8 followed by mxl_block_fp8_gemm.  One
 * row (K <= 8192): every wavefront of the GEMM quantizes its own super-tiles of it; more
 * rows: the producer waves, scratch slots and handoff of mxl_swiglu_mx_gemm, K % 128 == 0,
 * K <= 3584 or 4096 < K <= 7168.  Replaces the per-token-group quantization + block-FP8 GEMM pair
 * of the patched CutlassFp8BlockScaledMMKernel at decode sizes
 * (src/vllm_mach/fp8/linear.py:65-81,157-216). */
int mxl_block_fp8_quant_gemm(const void* x, int64_t M, int64_t K, const void* w_tiled, const void* sb, int64_t N,
                             const void* bias, void* out, int64_t ldc, void* stream);

/* mxl_block_fp8_quant_gemm with the output format and scale of `options`
 * (options->kernel -1 automatic, 0 the handoff, 3 the wavefronts' own quantization of one
 * row). */
int mxl_block_fp8_quant_gemm_ex(const void* x, int64_t M, int64_t K, const void* w_tiled, const void* sb, int64_t N,
                                const void* bias, void* out, int64_t ldc, const mxl_gemm_options* options,
                                void* stream);

/* 1 when the one-launch producer + GEMM runs (kind 0 mxl_swiglu_mx_gemm, 1
 * mxl_quant_mx_gemm, 2 mxl_block_fp8_quant_gemm; 3 mxl_quant_mx_gemm and 4
 * mxl_block_fp8_quant_gemm with the quantization in the GEMM's own wavefronts, the
 * scheme that measured faster than two launches) for M rows, K, scale rule and weight
 * format, else 0.  No counterpart in the reference (its fused rows are fixed,
 * src/vllm_mach/mxfp6/fused_mlp.py:13-19); for callers choosing between one launch and
 * two. */
int mxl_producer_gemm_supported(int kind, int64_t M, int64_t K, int rule, int w_fmt);

/* Block-FP8 GEMM: y[m, n] = sum_g sa[g*M + m] * sb[(n/128) * (K/128) + g] *
 * (A_g . W_g) with fp32 FMA per K128 block, bf16 out.  A E4M3 [M, K]; W tiled
 * E4M3 (fmt 0, no scales); sb fp32 [ceil(N/128), K/128].  Replaces
 * vllm_mach_block_fp8::mm / the ordered route / cutlass_scaled_mm
 * (src/vllm_mach/fp8/linear.py:65-81, src/vllm_mach/fp8/ordered.py:8-64,
 * native/block_fp8/block_fp8.cu:229-255). */
int mxl_block_fp8_gemm(const void* a, const void* sa_colmajor, int64_t M, const void* w_tiled,
                       const void* sb, int64_t N, int64_t K, const void* bias, void* out, int64_t ldc,
                       void* workspace, int64_t workspace_bytes, void* stream);

/* mxl_block_fp8_gemm with per-call options (kernel, splits, tiles; sa_layout
 * must be 0). */
int mxl_block_fp8_gemm_ex(const void* a, const void* sa_colmajor, int64_t M, const void* w_tiled, const void* sb,
                          int64_t N, int64_t K, const void* bias, void* out, int64_t ldc, void* workspace,
                          int64_t workspace_bytes, const mxl_gemm_options* options, void* stream);

/* Grouped MX GEMM over experts: output row p (bf16 [routed_rows, N]) of expert
 * e, expert_offsets[e] <= p < expert_offsets[e+1], is A[row_index[p] / row_div]
 * . W[e]^T (A[p] when row_index is NULL).  W: num_experts tiled weights laid
 * out back to back.  Replaces grouped_gemm_w6a8_out
 * (src/vllm_mach/mxfp6/moe_utils.py:320-380, src/vllm_mach/mxfp6/moe.py:671-696). */
int mxl_grouped_gemm(const void* a, const void* sa, int64_t a_rows, const int32_t* row_index, int row_div,
                     const int64_t* expert_offsets, int64_t num_experts, int64_t routed_rows,
                     const void* w_tiled, const void* sw_tiled, int64_t N, int64_t K, int w_fmt,
                     void* out, void* stream);

/* mxl_grouped_gemm with a per-call schedule (options->kernel: -1 automatic,
 * 0 16-row weight-streaming units, 3 96-row units, 1 wide 128-row tiles
 * (tile_m 4: 64-row), 2 per-expert generic). */
int mxl_grouped_gemm_ex(const void* a, const void* sa, int64_t a_rows, const int32_t* row_index, int row_div,
                        const int64_t* expert_offsets, int64_t num_experts, int64_t routed_rows,
                        const void* w_tiled, const void* sw_tiled, int64_t N, int64_t K, int w_fmt, void* out,
                        const mxl_gemm_options* options, void* stream);

/* Grouped GEMMs with the activation producer fused (one launch instead of two):
 * each workgroup computes its rows' MXFP8 operands in LDS with the standalone
 * producers' arithmetic, so the output is bit-identical to the two-call path.
 *   _quant:  A = MXFP8(x[row_index[p] / row_div]) under `rule` (x bf16, row stride
 *            ldx), as mxl_quantize_mxfp8 then mxl_grouped_gemm;
 *   _swiglu: A = SwiGLU -> MXFP8 of gate_up bf16 [routed_rows, 2K] (gate columns
 *            [0, K), up [K, 2K)) under `rule`, as mxl_swiglu_mxfp8 then
 *            mxl_grouped_gemm; replaces silu_and_mul_mxfp8_grouped +
 *            grouped_gemm_w6a8_out (mxfp6_sm120_silu_grouped_gemm,
 *            src/vllm_mach/mxfp6/moe_utils.py:383-442).
 * They run the weight-streaming grouped schedule of 16-row units (below 32
 * routed rows per expert on average, the operands of a unit within 64 KiB of
 * LDS); mxl_grouped_fused_supported says whether a shape has one, and the entry
 * points return MXL_EUNSUPPORTED otherwise.  Replace the fused
 * router/quant and SiLU schedules of src/vllm_mach/mxfp6/moe.py:126-190. */
int mxl_grouped_fused_supported(int64_t routed_rows, int64_t num_experts, int64_t K, int w_fmt);
int mxl_grouped_gemm_quant(const void* x, int64_t ldx, const int32_t* row_index, int row_div,
                           const int64_t* expert_offsets, int64_t num_experts, int64_t routed_rows,
                           const void* w_tiled, const void* sw_tiled, int64_t N, int64_t K, int w_fmt, int rule,
                           void* out, void* stream);
int mxl_grouped_gemm_swiglu(const void* gate_up, const int64_t* expert_offsets, int64_t num_experts,
                            int64_t routed_rows, const void* w_tiled, const void* sw_tiled, int64_t N, int64_t K,
                            int w_fmt, int rule, void* out, void* stream);

/* Down projection with the weighted combine in the same launch.  The routed
 * rows are computed as mxl_grouped_gemm (row_index NULL: row p of A is routed
 * row p; else A[row_index[p] / row_div]) or mxl_grouped_gemm_swiglu compute them and stored into routed_out
 * (bf16 [routed_rows, N]); each token's row out[t] = bf16(sum over k ascending
 * of topk_weights[t, k] * routed_out[inverse[t * topk + k]]) in fp32 -- the
 * arithmetic of mxl_moe_reduce, so out is bit-identical to the GEMM followed by
 * mxl_moe_reduce -- is written by the workgroup that stores the token's last
 * routed row (a per-token device-scope atomic counter; the routed rows are
 * stored and read device-coherently, the count taken after the stores complete).
 * Tokens whose routes are all dropped get a zero row.  counters: int32 [T], zero
 * before the first call; every call leaves them zero, so calls that share
 * counters must not overlap (one set per stream).  They run the
 * small-batch schedule (16-row weight-streaming units: fewer than 32 routed rows
 * per expert) at K <= 512, topk <= 16 and routed_rows * N * 2 below 2 GiB;
 * mxl_grouped_combine_supported says whether a shape has one (prod 0: plain
 * MXFP8 operands, 2: the SwiGLU producer) and the entry points return
 * MXL_EUNSUPPORTED otherwise.  Replace grouped_gemm_w6a8_out + moe_reduce_out
 * (src/vllm_mach/mxfp6/moe.py:671-702) in one launch, as the reference's
 * qwen35_w2_splitk_reduce_out / array_gemm_w6a8_reduce_out fold the combine
 * into w2 (src/vllm_mach/mxfp6/moe.py:163-186). */
typedef struct mxl_moe_combine {
  const int32_t* sorted_routes; /* [routed_rows]: route t * topk + k of routed row p */
  const int32_t* inverse;       /* [T * topk]: routed row of route (t, k), -1 if dropped */
  const float* topk_weights;    /* fp32 [T, topk] */
  int64_t T;
  int64_t topk;                 /* 1 .. 16 */
  void* out;                    /* bf16 [T, N] */
  int32_t* counters;            /* int32 [T], zero; left zero */
} mxl_moe_combine;
int mxl_grouped_combine_supported(int64_t routed_rows, int64_t num_experts, int64_t N, int64_t K, int w_fmt,
                                  int prod);
int mxl_grouped_gemm_combine(const void* a, const void* sa, int64_t a_rows, const int32_t* row_index, int row_div,
                             const int64_t* expert_offsets, int64_t num_experts, int64_t routed_rows,
                             const void* w_tiled, const void* sw_tiled, int64_t N, int64_t K, int w_fmt,
                             void* routed_out, const mxl_moe_combine* combine, void* stream);
int mxl_grouped_gemm_swiglu_combine(const void* gate_up, const int64_t* expert_offsets, int64_t num_experts,
                                    int64_t routed_rows, const void* w_tiled, const void* sw_tiled, int64_t N,
                                    int64_t K, int w_fmt, int rule, void* routed_out,
                                    const mxl_moe_combine* combine, void* stream);

/* Token sort by expert (stable): topk_ids int32 [T, topk] -> sorted_routes
 * int32 [T*topk], expert_offsets int64 [E+1], inverse int32 [T*topk] (-1 for
 * ids outside [0, E)).  1 <= E <= 2560.  Replaces route_mxfp8_out's routing outputs
 * (src/vllm_mach/mxfp6/moe_utils.py:205-255, src/vllm_mach/mxfp6/moe.py:651-669). */
int64_t mxl_moe_route_workspace_bytes(int64_t T, int64_t topk, int64_t E);
int mxl_moe_route(const int32_t* topk_ids, int64_t T, int64_t topk, int64_t E, int32_t* sorted_routes,
                  int64_t* expert_offsets, int32_t* inverse, void* workspace, int64_t workspace_bytes,
                  void* stream);

/* Router: softmax -> top-k -> (renormalize) from router logits [T, E] (fp32, or bf16
 * with logits_bf16 = 1) and the token sort of mxl_moe_route, for E <= 1024 and
 * topk <= min(E, 64).  topk_ids int32 [T, topk] are the k largest logits of each token
 * (softmax is increasing in the logit) in descending order, ties to the lower expert
 * index (-0 equals +0; NaNs order by sign beyond the finite values);
 * topk_weights fp32 [T, topk] = exp(x - max) / sum, the sum over the selected experts
 * (renormalize = 1) or over all experts (0), with this library's binary32 exp.  Then
 * sorted_routes / expert_offsets / inverse exactly as mxl_moe_route writes them for
 * those ids.  One launch while T * topk <= 1024; two while topk divides 1024 and the
 * chunk histograms fit one workgroup; otherwise the routing and mxl_moe_route's
 * launches.  Replaces vLLM's fused top-k softmax (select_experts: softmax, topk,
 * renormalize) and the routing of route_mxfp8_out, fused as the reference's
 * qwen35_router_quant_out fuses them (src/vllm_mach/mxfp6/moe.py:142-152). */
int64_t mxl_moe_router_workspace_bytes(int64_t T, int64_t topk, int64_t E);
int mxl_moe_router(const void* logits, int logits_bf16, int64_t T, int64_t E, int64_t topk, int renormalize,
                   float* topk_weights, int32_t* topk_ids, int32_t* sorted_routes, int64_t* expert_offsets,
                   int32_t* inverse, void* workspace, int64_t workspace_bytes, void* stream);

/* Weighted combine: out[t, h] = bf16(sum_k y[inverse[t*topk+k], h] * w[t, k])
 * in fp32, k ascending.  Replaces moe_reduce_out
 * (src/vllm_mach/mxfp6/moe.py:697-702, src/vllm_mach/mxfp6/moe_utils.py:445-488). */
int mxl_moe_reduce(const void* routed_output, const float* topk_weights, const int32_t* inverse, int64_t T,
                   int64_t topk, int64_t H, void* out, void* stream);

/* The same combine with a bf16 addend [T, H] (a shared expert's output) added to
 * the fp32 sum after the routes, before the one rounding: out[t, h] =
 * bf16(sum_k y[...] * w[t, k] + addend[t, h]).  Replaces the shared-output form of
 * qwen35_grouped_reduce_out (src/vllm_mach/mxfp6/moe.py:301-302). */
int mxl_moe_reduce_add(const void* routed_output, const float* topk_weights, const int32_t* inverse, int64_t T,
                       int64_t topk, int64_t H, const void* addend, void* out, void* stream);

/* The kernels a dense GEMM call (mxl_mx_gemm_ex, block = 0; mxl_block_fp8_gemm_ex,
 * block = 1) or a grouped GEMM call (mxl_grouped_gemm_ex, prod = 0;
 * mxl_grouped_gemm_quant, prod = 1; mxl_grouped_gemm_swiglu, prod = 2) launches
 * for a shape and options, named as the profiler prints them (template arguments
 * without spaces) and joined by " + ", written NUL-terminated into buf[len].  No
 * counterpart in the reference: a diagnostic for matching profiles to the kernels
 * that run (the plan assumes a workspace large enough for the K split). */
int mxl_gemm_plan_name(int64_t M, int64_t N, int64_t K, int w_fmt, int block, const mxl_gemm_options* options,
                       char* buf, int64_t len);
int mxl_grouped_plan_name(int64_t routed_rows, int64_t num_experts, int64_t K, int w_fmt, int prod, int rule,
                          const mxl_gemm_options* options, char* buf, int64_t len);

#ifdef __cplusplus
}
#endif

#endif /* MXLINEAR_H */
