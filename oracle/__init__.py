"""CPU oracle for the quantized-linear hot path (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker: the product path in
``vllm-mach_amd/`` never imports it and fails loudly without its HIP library.

The bit-level algorithms live in ``mx_oracle.c`` (binary32, round-to-nearest-
even, no FMA contraction) and are loaded through ctypes; the contractions are
numpy float64 matmuls over exactly dequantized operands.  Each wrapper names
the reference function it restates (troycheng/vllm-mach v0.4.0, file:line).

Pinning (what checks each function, beyond retyping its formula) is listed in
the test modules ``tests/test_oracle_*.py``.  Functions without a reference
vector or an independent mathematical check say "parity unpinned" below.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libmxoracle.so"
SOURCE = HERE / "mx_oracle.c"

FMT_E4M3, FMT_E2M3, FMT_E3M2 = 0, 2, 3
RULE_FLOOR_CARRY175, RULE_CEIL_DIV448, RULE_RP_UE8M0 = 0, 1, 2

_lib = None


def build(force: bool = False) -> Path:
    """Compile the C restatement with gcc (IEEE binary32, no contraction)."""
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < SOURCE.stat().st_mtime:
        tmp = LIB_PATH.with_suffix(".so.tmp")
        subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math",
                        "-fPIC", "-shared", str(SOURCE), "-o", str(tmp), "-lm"], check=True)
        os.replace(tmp, LIB_PATH)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        I = ctypes.c_int
        sig = {
            "mxo_f32_to_e4m3": (ctypes.c_uint8, [ctypes.c_float]),
            "mxo_e4m3_to_f32": (ctypes.c_float, [ctypes.c_uint8]),
            "mxo_f32_to_fp6": (ctypes.c_uint8, [ctypes.c_float, I]),
            "mxo_fp6_to_f32": (ctypes.c_float, [ctypes.c_uint8, I]),
            "mxo_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "mxo_exp": (ctypes.c_float, [ctypes.c_float]),
            "mxo_pack_fp6": (None, [P, I64, P]),
            "mxo_unpack_fp6": (None, [P, I64, P]),
            "mxo_quant_mxfp8": (None, [P, I64, I64, I, P, P]),
            "mxo_swiglu_mxfp8": (None, [P, I64, I64, I, P, P]),
            "mxo_swizzle_offset": (I64, [I64, I64, I64]),
            "mxo_swizzle_size": (I64, [I64, I64]),
            "mxo_swizzle_scales": (None, [P, I64, I64, P]),
            "mxo_quant_block_fp8": (None, [P, I64, I64, P, P]),
            "mxo_silu_mul_block_fp8": (None, [P, I64, I64, I, P, P]),
            "mxo_block_fp8_ordered_reduce": (None, [P, P, P, I64, I64, I64, P]),
            "mxo_quant_mxfp6": (None, [P, I64, I64, I, P, P]),
            "mxo_dequant_mx": (None, [P, P, I64, I64, I, P]),
            "mxo_moe_route": (None, [P, I64, I64, I64, P, P, P]),
            "mxo_moe_reduce": (None, [P, P, P, I64, I64, I64, P]),
            "mxo_rmsnorm_mx": (None, [P, P, P, I64, I64, ctypes.c_float, I, P, P, P, P]),
            "mxo_quant_mxfp8_dual": (None, [P, I64, I64, I, P, P, P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------ bf16 I/O

def bf16_bits(x) -> np.ndarray:
    """bf16 torch tensor (any device) or uint16 array -> contiguous uint16 numpy."""
    if isinstance(x, np.ndarray):
        assert x.dtype == np.uint16
        return np.ascontiguousarray(x)
    import torch
    assert x.dtype == torch.bfloat16
    return np.ascontiguousarray(x.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16))


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even binary32 -> bf16 bits (NaN -> 0x7FC0)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    out = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    out[nan] = 0x7FC0
    return out


# --------------------------------------------------------------- codecs

_E4M3_LUT = None


def e4m3_to_f32(codes: np.ndarray) -> np.ndarray:
    global _E4M3_LUT
    if _E4M3_LUT is None:
        L = lib()
        _E4M3_LUT = np.array([L.mxo_e4m3_to_f32(i) for i in range(256)], dtype=np.float32)
    return _E4M3_LUT[codes]


def f32_to_e4m3_scalar(v: float) -> int:
    return lib().mxo_f32_to_e4m3(float(v))


def fp6_to_f32(codes: np.ndarray, fmt: int) -> np.ndarray:
    L = lib()
    lut = np.array([L.mxo_fp6_to_f32(i, fmt) for i in range(64)], dtype=np.float32)
    return lut[codes & 63]


def pack_fp6(codes: np.ndarray) -> np.ndarray:
    """[..., K] 6-bit codes -> [..., 3K/4] bytes (4 values per 3 bytes, LE bit stream)."""
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(codes.shape[:-1] + (codes.shape[-1] * 3 // 4,), dtype=np.uint8)
    lib().mxo_pack_fp6(_p(codes), codes.size, _p(out))
    return out


def unpack_fp6(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 4 // 3,), dtype=np.uint8)
    lib().mxo_unpack_fp6(_p(packed), out.size, _p(out))
    return out


def exp_f32(x: np.ndarray) -> np.ndarray:
    L = lib()
    return np.array([L.mxo_exp(float(v)) for v in np.asarray(x, dtype=np.float32).ravel()],
                    dtype=np.float32).reshape(np.shape(x))


# ----------------------------------------------------------- quantizers

def quant_mxfp8(x, rule: int = RULE_FLOOR_CARRY175):
    """bf16 [R, K] -> (E4M3 codes [R, K] u8, E8M0 scales [R, K/32] u8).

    rule 0 restates ``quantize_block`` (src/vllm_mach/mxfp8/reconstruct_model.py:34-50);
    rule 1 is the ``ceil_div448`` E8M0 rule of mxfp6/mxfp8_mlp.py:100-105;
    rule 2 (``rp_ue8m0``) is FlashInfer's ``mxfp8_quantize`` convention as
    src/vllm_mach/mxfp8/swiglu_quant.py:58-66 writes it (1/448 correctly rounded).
    """
    b = bf16_bits(x)
    R, K = b.shape
    assert K % 32 == 0
    codes = np.empty((R, K), np.uint8)
    scales = np.empty((R, K // 32), np.uint8)
    lib().mxo_quant_mxfp8(_p(b), R, K, rule, _p(codes), _p(scales))
    return codes, scales


def quant_mxfp8_dual(x, rule: int = RULE_FLOOR_CARRY175):
    """Two-limb MXFP8 (src/vllm_mach/mxfp8/dual.py:45-50): bf16 [R, K] -> (hi codes, hi
    scales, residual codes, residual scales), each [R, K] / [R, K/32]."""
    b = bf16_bits(x)
    R, K = b.shape
    hi = np.empty((R, K), np.uint8); s_hi = np.empty((R, K // 32), np.uint8)
    res = np.empty((R, K), np.uint8); s_res = np.empty((R, K // 32), np.uint8)
    lib().mxo_quant_mxfp8_dual(_p(b), R, K, rule, _p(hi), _p(s_hi), _p(res), _p(s_res))
    return hi, s_hi, res, s_res


def swiglu_mxfp8(gate_up, rule: int = RULE_CEIL_DIV448):
    """bf16 [R, 2K] -> codes [R, K], logical scales [R, K/32] (mxfp6/mxfp8_mlp.py:87-110;
    rule 2: the single-rounding champion variant, mxfp8/swiglu_quant.py:54-66)."""
    b = bf16_bits(gate_up)
    R, K2 = b.shape
    K = K2 // 2
    codes = np.empty((R, K), np.uint8)
    scales = np.empty((R, K // 32), np.uint8)
    lib().mxo_swiglu_mxfp8(_p(b), R, K, rule, _p(codes), _p(scales))
    return codes, scales


def rmsnorm_mx(x, residual, weight, eps: float, rule: int = RULE_CEIL_DIV448, quant: bool = True):
    """Residual add + Gemma RMSNorm (+ MXFP8) per row (mxfp6/mxfp8_norm_quant.py:15-39,
    mxfp6/gemma_norm.py:13-29).  x, residual bf16 [R, N] (residual may be None), weight
    bf16 [N].  Returns (codes [R, N], logical scales [R, N/32], summed bf16 bits [R, N]) when
    `quant`, else (y bf16 bits [R, N], summed bf16 bits [R, N])."""
    xb = bf16_bits(x)
    R, N = xb.shape
    rb = bf16_bits(residual) if residual is not None else None
    wb = bf16_bits(weight).reshape(-1)
    assert wb.shape[0] == N and N % 32 == 0
    summed = np.empty((R, N), np.uint16)
    if quant:
        codes = np.empty((R, N), np.uint8)
        scales = np.empty((R, N // 32), np.uint8)
        lib().mxo_rmsnorm_mx(_p(xb), _p(rb) if rb is not None else None, _p(wb), R, N, eps, rule,
                             _p(codes), _p(scales), _p(summed), None)
        return codes, scales, summed
    y = np.empty((R, N), np.uint16)
    lib().mxo_rmsnorm_mx(_p(xb), _p(rb) if rb is not None else None, _p(wb), R, N, eps, rule,
                         None, None, _p(summed), _p(y))
    return y, summed


def swizzle_offset(r: int, g: int, K: int) -> int:
    return lib().mxo_swizzle_offset(r, g, K)


def swizzle_scales(logical: np.ndarray, K: int) -> np.ndarray:
    """Logical [R, K/32] -> flat swizzled buffer (mxfp8_mlp.py:107-110,122); padding = 0."""
    logical = np.ascontiguousarray(logical, dtype=np.uint8)
    R = logical.shape[0]
    out = np.zeros(lib().mxo_swizzle_size(R, K), np.uint8)
    lib().mxo_swizzle_scales(_p(logical), R, K, _p(out))
    return out


def quant_block_fp8(x):
    """bf16 [M, K] -> (E4M3 [M, K], fp32 scales [M, K/128] column-major data).

    Restates fp8/_quantize_kernel.py:8-18.  The scale array is returned as
    numpy with shape [M, K/128] whose memory is column-major (Fortran order).
    """
    b = bf16_bits(x)
    M, K = b.shape
    q = np.empty((M, K), np.uint8)
    s = np.empty((K // 128) * M, np.float32)
    lib().mxo_quant_block_fp8(_p(b), M, K, _p(q), _p(s))
    return q, s.reshape(K // 128, M).T


def silu_mul_block_fp8(x, transposed: bool = False):
    """bf16 [R, 2H] -> (E4M3 [R, H], fp32 scales [R, H/128]) per native/fp8_activation/activation.cu:18-60."""
    b = bf16_bits(x)
    R, H2 = b.shape
    H = H2 // 2
    q = np.empty((R, H), np.uint8)
    s = np.empty(R * (H // 128), np.float32)
    lib().mxo_silu_mul_block_fp8(_p(b), R, H, int(transposed), _p(q), _p(s))
    s = s.reshape(H // 128, R).T if transposed else s.reshape(R, H // 128)
    return q, s


def quant_mxfp6(x, fmt: int = FMT_E2M3):
    """bf16 [R, K] -> (unpacked 6-bit codes [R, K], E8M0 scales [R, K/32]).

    OCP MX v1.0 floor rule.  The reference's MXFP6 weights come from an external
    offline quantizer with no vectors in the tree: parity unpinned against the
    reference; pinned against the OCP definition by brute force in the tests.
    """
    b = bf16_bits(x)
    R, K = b.shape
    codes = np.empty((R, K), np.uint8)
    scales = np.empty((R, K // 32), np.uint8)
    lib().mxo_quant_mxfp6(_p(b), R, K, fmt, _p(codes), _p(scales))
    return codes, scales


def dequant_mx(codes: np.ndarray, scales: np.ndarray, fmt: int) -> np.ndarray:
    """codes [R, K] (FP6 unpacked) + E8M0 [R, K/32] -> exact fp32 values."""
    codes = np.ascontiguousarray(codes, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint8)
    R, K = codes.shape
    out = np.empty((R, K), np.float32)
    lib().mxo_dequant_mx(_p(codes), _p(scales), R, K, fmt, _p(out))
    return out


# ------------------------------------------------------------- GEMM refs

def mx_gemm_ref(a_codes, a_scales, w_codes, w_scales, w_fmt: int = FMT_E4M3,
                a_fmt: int = FMT_E4M3) -> np.ndarray:
    """Dequantize-then-matmul (tests/native_mxfp6/test_mxfp8_sm120.py:53-57), float64
    accumulation of exactly dequantized operands; returns fp32 [M, N] (round to
    bf16 with ``f32_to_bf16``)."""
    a = dequant_mx(a_codes, a_scales, a_fmt).astype(np.float64)
    w = dequant_mx(w_codes, w_scales, w_fmt).astype(np.float64)
    return (a @ w.T).astype(np.float32)


def block_fp8_gemm_ref(a_q, sa, w_q, sb) -> np.ndarray:
    """Block-FP8 ordered route (fp8/ordered.py:8-64): exact per-K128 partial dots,
    then ascending-g fp32 FMA with sa*sb, one bf16 rounding.  Returns bf16 bits.

    a_q E4M3 [M, K]; sa fp32 [M, K/128]; w_q E4M3 [N, K]; sb fp32 [N/128, K/128].
    """
    M, K = a_q.shape
    N = w_q.shape[0]
    G = K // 128
    a = e4m3_to_f32(a_q).astype(np.float64)
    w = e4m3_to_f32(w_q).astype(np.float64)
    raw = np.empty((G, M, N), np.float32)
    for g in range(G):
        raw[g] = a[:, g * 128:(g + 1) * 128] @ w[:, g * 128:(g + 1) * 128].T
    sa_col = np.ascontiguousarray(np.asarray(sa, np.float32).T)      # [G, M]
    sb_c = np.ascontiguousarray(sb, np.float32)
    out = np.empty((M, N), np.uint16)
    lib().mxo_block_fp8_ordered_reduce(_p(raw), _p(sa_col), _p(sb_c), M, N, G, _p(out))
    return out


# ------------------------------------------------------------------- MoE

def moe_route(topk_ids: np.ndarray, num_experts: int):
    """Stable token sort (contract of route_mxfp8_out, mxfp6/moe_utils.py:205-255)."""
    ids = np.ascontiguousarray(topk_ids, np.int32)
    T, topk = ids.shape
    sorted_routes = np.full(T * topk, -1, np.int32)
    offsets = np.empty(num_experts + 1, np.int64)
    inverse = np.empty(T * topk, np.int32)
    lib().mxo_moe_route(_p(ids), T, topk, num_experts, _p(sorted_routes), _p(offsets), _p(inverse))
    return sorted_routes, offsets, inverse


def order_keys(logits) -> np.ndarray:
    """Binary32 logits as unsigned keys in value order (-0 read as +0; NaNs beyond the
    finite values by sign): the total order the router selects by."""
    u = np.ascontiguousarray(np.asarray(logits, np.float32)).view(np.uint32).copy()
    u[u == 0x80000000] = 0
    neg = (u & 0x80000000) != 0
    return np.where(neg, ~u, u | np.uint32(0x80000000)).astype(np.uint32)


def moe_router(logits, top_k: int, renormalize: bool = True):
    """softmax -> top-k -> (renormalize) -> token sort (vLLM's select_experts, the routing
    half of qwen35_router_quant_out, src/vllm_mach/mxfp6/moe.py:142-152; vLLM's top-k softmax
    kernel breaks ties to the lower expert).  ids: the k largest logits of each token,
    descending, ties to the lower index (softmax is increasing, so these are its k
    largest probabilities); weights: exp(x - max) / sum in float64, the sum over the
    selected experts (renormalize) or all experts.  Returns (weights float64 [T, k],
    ids int32 [T, k], sorted_routes, expert_offsets, inverse)."""
    x = np.ascontiguousarray(np.asarray(logits, np.float32))
    T, E = x.shape
    keys = order_keys(x).astype(np.int64)
    # descending key, ascending index: a stable sort of the negated keys
    ids = np.argsort(-keys, axis=1, kind="stable")[:, :top_k].astype(np.int32)
    xd = x.astype(np.float64)
    top = np.take_along_axis(xd, ids[:, :1].astype(np.int64), axis=1)
    e_sel = np.exp(np.take_along_axis(xd, ids.astype(np.int64), axis=1) - top)
    denom = e_sel.sum(axis=1, keepdims=True) if renormalize else np.exp(xd - top).sum(axis=1, keepdims=True)
    weights = e_sel / denom
    sorted_routes, offsets, inverse = moe_route(ids, E)
    return weights, ids, sorted_routes, offsets, inverse


def moe_reduce(y_bits: np.ndarray, topk_weights: np.ndarray, inverse: np.ndarray) -> np.ndarray:
    """out[t] = bf16(sum_k w[t,k] * y[inverse[t*topk+k]]) (mxfp6/moe.py:697-702)."""
    y_bits = np.ascontiguousarray(y_bits, np.uint16)
    w = np.ascontiguousarray(topk_weights, np.float32)
    inv = np.ascontiguousarray(inverse, np.int32)
    T, topk = w.shape
    H = y_bits.shape[1]
    out = np.empty((T, H), np.uint16)
    lib().mxo_moe_reduce(_p(y_bits), _p(w), _p(inv), T, topk, H, _p(out))
    return out


def moe_ref(hidden, w13_codes, w13_scales, w2_codes, w2_scales, topk_weights, topk_ids,
            fmt: int = FMT_E2M3, act_rule: int = RULE_FLOOR_CARRY175,
            mid_rule: int = RULE_CEIL_DIV448) -> np.ndarray:
    """Per-expert dense MoE reference (tests/native_mxfp6/test_moe.py:230-247).

    hidden bf16 [T, H] -> MXFP8; per expert e: gate_up = bf16(A @ W13[e]^T);
    SwiGLU with bf16 SiLU then MXFP8 (``swiglu_mxfp8``); y = bf16(. @ W2[e]^T);
    weighted combine in fp32 over k ascending.  Weight codes are unpacked.
    Returns bf16 bits [T, H].
    """
    hb = bf16_bits(hidden)
    T, H = hb.shape
    ids = np.asarray(topk_ids, np.int32)
    E = w13_codes.shape[0]
    a_codes, a_scales = quant_mxfp8(hb, act_rule)
    sorted_routes, offsets, inverse = moe_route(ids, E)
    topk = ids.shape[1]
    y = np.zeros((T * topk, H), np.uint16)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if lo == hi:
            continue
        toks = sorted_routes[lo:hi] // topk
        g = mx_gemm_ref(a_codes[toks], a_scales[toks], w13_codes[e], w13_scales[e], fmt)
        gu = f32_to_bf16(g)
        c2, s2 = swiglu_mxfp8(gu, mid_rule)
        y[lo:hi] = f32_to_bf16(mx_gemm_ref(c2, s2, w2_codes[e], w2_scales[e], fmt))
    return moe_reduce(y, np.asarray(topk_weights, np.float32), inverse)
