"""Pins of the oracle's residual + Gemma RMSNorm (+ MXFP8) producer
(src/vllm_mach/mxfp6/mxfp8_norm_quant.py:15-39, src/vllm_mach/mxfp6/gemma_norm.py:13-29)
by what the arithmetic fixes independently of the restatement:

* summed is torch's bf16 rounding of the fp32 sum x + residual, bit for bit;
* y agrees with a float64 evaluation of the normalization to half a bf16 ulp except at
  rounding ties that the binary32 path decides the other way;
* the MXFP8 step applied to the oracle's own y, evaluated with torch's float8 cast and
  the ceil_div448 exponent rule (mxfp8_norm_quant.py:27-33), gives the same codes and
  scales;
* closed forms: a zero row gives scale 28 and zero codes; a constant row normalizes to
  +-1, whose E4M3 code at scale 2^-8 is 0x78 / 0xF8.
"""
import numpy as np
import torch

import oracle


def _case(R, N, seed, residual=True, wstd=0.2):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(R, N, generator=g).bfloat16()
    r = (torch.randn(R, N, generator=g) * 3).bfloat16() if residual else None
    w = (torch.randn(N, generator=g) * wstd).bfloat16()
    return x, r, w


def _y64(x, r, w, eps):
    s = x.double() + (r.double() if r is not None else 0)
    return s * torch.rsqrt((s * s).mean(-1, keepdim=True) + eps) * (w.double() + 1)


def test_summed_is_bf16_of_fp32_sum():
    x, r, w = _case(5, 2560, 1)
    _, _, summed = oracle.rmsnorm_mx(x, r, w, 1e-6)
    ref = oracle.bf16_bits((x.float() + r.float()).bfloat16())
    assert np.array_equal(summed, ref)


def test_y_matches_float64_normalization():
    for residual in (True, False):
        x, r, w = _case(9, 5120, 2, residual)
        y, _ = oracle.rmsnorm_mx(x, r, w, 1e-6, quant=False)
        got = oracle.bf16_to_f32(y).astype(np.float64)
        ref = _y64(x, r, w, 1e-6).numpy()
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
        err = np.abs(got - ref) / ulp
        assert err.max() <= 1.0 + 1e-6
        assert (err <= 0.5 + 1e-3).mean() > 0.995


def test_codes_follow_ceil_div448_of_y():
    x, r, w = _case(6, 2048, 3)
    codes, scales, _ = oracle.rmsnorm_mx(x, r, w, 1e-6, oracle.RULE_CEIL_DIV448)
    y, _ = oracle.rmsnorm_mx(x, r, w, 1e-6, quant=False)
    yt = torch.from_numpy(oracle.bf16_to_f32(y)).view(6, 64, 32)
    raw = torch.clamp(yt.abs().amax(-1) / 448.0, min=1e-30)
    bits = (raw.view(torch.int32) + 0x7FFFFF) & 0x7F800000
    assert np.array_equal(scales, (bits >> 23).numpy().astype(np.uint8))
    q = (yt * (1.0 / bits.view(torch.float32))[..., None]).to(torch.float8_e4m3fn)
    assert np.array_equal(codes, q.view(torch.uint8).reshape(6, 2048).numpy())


def test_zero_and_constant_rows():
    N = 256
    x = torch.zeros(2, N).bfloat16()
    x[1] = 1.0
    x[1, ::2] = -1.0
    w = torch.zeros(N).bfloat16()
    codes, scales, _ = oracle.rmsnorm_mx(x, None, w, 1e-6)
    assert (scales[0] == 28).all() and (codes[0] == 0).all()
    assert (scales[1] == 119).all()
    assert (codes[1, ::2] == 0xF8).all() and (codes[1, 1::2] == 0x78).all()


def test_variance_order_is_a_sum():
    """The fixed butterfly order only reassociates: the oracle's y equals the y computed
    from a float64 variance except where the binary32 sum lands on the other side of a
    rounding boundary (rare)."""
    x, r, w = _case(4, 16384, 4)
    y, _ = oracle.rmsnorm_mx(x, r, w, 1e-5, quant=False)
    s = x.float() + r.float()
    var64 = (s.double() ** 2).mean(-1, keepdim=True).float()
    rs = 1.0 / torch.sqrt(var64 + 1e-5)
    y2 = ((s * rs) * (w.float() + 1)).bfloat16()
    assert (oracle.bf16_bits(y2) == y).mean() > 0.999
