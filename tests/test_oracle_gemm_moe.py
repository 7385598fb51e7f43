"""Pin the oracle's GEMM, block-FP8 ordered reduction and MoE references.

* dequantize-then-matmul: torch's float8 decode and an fp64 matmul (the pattern of
  tests/native_mxfp6/test_mxfp8_sm120.py:53-57).
* block-FP8 ordered route: the unordered fp64 sum of sa*sb*dot (fp8/ordered.py:8-64
  only fixes the order, so the two must agree to fp32 rounding).
* token sort: numpy's stable argsort; weighted combine: the reference test's torch
  expression (tests/native_mxfp6/test_moe.py:243-247), bit for bit.
* MoE: a per-token loop (different loop nest than the per-expert reference).
"""
import numpy as np
import torch


def test_mx_gemm_ref_matches_torch_dequant(oracle_mod):
    g = torch.Generator().manual_seed(29)
    a = torch.randn(7, 512, generator=g).bfloat16()
    w = (torch.randn(40, 512, generator=g) * 0.02).bfloat16()
    ac, as_ = oracle_mod.quant_mxfp8(a)
    wc, ws = oracle_mod.quant_mxfp8(w)
    got = oracle_mod.mx_gemm_ref(ac, as_, wc, ws)
    ta = torch.from_numpy(ac).view(torch.float8_e4m3fn).double() * torch.exp2(
        torch.from_numpy(as_).double() - 127).repeat_interleave(32, 1)
    tw = torch.from_numpy(wc).view(torch.float8_e4m3fn).double() * torch.exp2(
        torch.from_numpy(ws).double() - 127).repeat_interleave(32, 1)
    ref = (ta @ tw.T).float().numpy()
    assert np.array_equal(got, ref)


def test_mxfp6_dequant_uses_packed_values(oracle_mod):
    g = torch.Generator().manual_seed(17)
    w = (torch.randn(16, 128, generator=g) * 0.1).bfloat16()
    for fmt in (2, 3):
        codes, scales = oracle_mod.quant_mxfp6(w, fmt)
        packed = oracle_mod.pack_fp6(codes)
        assert packed.shape == (16, 96)
        deq = oracle_mod.dequant_mx(oracle_mod.unpack_fp6(packed), scales, fmt)
        rel = np.linalg.norm(deq - w.float().numpy()) / np.linalg.norm(w.float().numpy())
        assert rel < (0.05 if fmt == 2 else 0.1)


def test_block_fp8_ordered_ref(oracle_mod):
    g = torch.Generator().manual_seed(173)
    M, N, K = 5, 256, 512
    x = torch.randn(M, K, generator=g).bfloat16()
    aq, sa = oracle_mod.quant_block_fp8(x)
    wq = (torch.randn(N, K, generator=g) * 0.02).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    sb = np.abs(np.random.default_rng(1).standard_normal((N // 128, K // 128))).astype(np.float32) + 0.5
    out = oracle_mod.block_fp8_gemm_ref(aq, sa, wq, sb)
    a = oracle_mod.e4m3_to_f32(aq).astype(np.float64)
    w = oracle_mod.e4m3_to_f32(wq).astype(np.float64)
    ref = np.zeros((M, N))
    for gi in range(K // 128):
        sl = slice(gi * 128, gi * 128 + 128)
        ref += (a[:, sl] @ w[:, sl].T) * sa[:, gi:gi + 1] * np.repeat(sb[:, gi], 128)[None, :]
    got = oracle_mod.bf16_to_f32(out)
    assert np.abs(got - ref).max() <= 2 ** -7 * np.abs(ref).max()
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 3e-3


def test_route_is_stable_counting_sort(oracle_mod):
    rng = np.random.default_rng(0)
    for T, topk, E in [(7, 2, 4), (128, 8, 256), (2048, 8, 256)]:
        ids = np.stack([rng.permutation(E)[:topk] for _ in range(T)]).astype(np.int32)
        sorted_routes, offsets, inverse = oracle_mod.moe_route(ids, E)
        order = np.argsort(ids.ravel(), kind="stable")
        assert np.array_equal(sorted_routes, order)
        assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(np.bincount(ids.ravel(), minlength=E))]))
        assert np.array_equal(inverse[order], np.arange(T * topk))
    ids = np.array([[0, 5], [-1, 1]], np.int32)  # out-of-range ids are dropped
    s, o, inv = oracle_mod.moe_route(ids, 2)
    assert o.tolist() == [0, 1, 2] and inv.tolist() == [0, -1, -1, 1]


def test_reduce_matches_reference_expression(oracle_mod):
    g = torch.Generator().manual_seed(12035)
    T, topk, H = 7, 2, 256
    y = torch.randn(T * topk, H, generator=g).bfloat16()
    w = torch.rand(T, topk, generator=g)
    w /= w.sum(-1, keepdim=True)
    inverse = torch.randperm(T * topk, generator=g).int()
    got = oracle_mod.moe_reduce(oracle_mod.bf16_bits(y), w.numpy(), inverse.numpy())
    rows = y[inverse.long()].reshape(T, topk, H)
    ref = sum(rows[:, k].float() * w[:, k, None] for k in range(topk)).bfloat16()
    assert np.array_equal(got, oracle_mod.bf16_bits(ref))


def test_moe_ref_matches_per_token_loop(oracle_mod):
    g = torch.Generator().manual_seed(12035)
    E, H, I, T, topk = 4, 256, 128, 7, 2
    w13 = (torch.randn(E, 2 * I, H, generator=g) * 0.1).bfloat16()
    w2 = (torch.randn(E, H, I, generator=g) * 0.1).bfloat16()
    q13 = [oracle_mod.quant_mxfp6(w13[e], 2) for e in range(E)]
    q2 = [oracle_mod.quant_mxfp6(w2[e], 2) for e in range(E)]
    c13 = np.stack([c for c, _ in q13]); s13 = np.stack([s for _, s in q13])
    c2 = np.stack([c for c, _ in q2]); s2 = np.stack([s for _, s in q2])
    x = torch.randn(T, H, generator=g).bfloat16()
    ids = np.array([[(j) % E, (j + 1) % E] for j in range(T)], np.int32)
    wts = torch.rand(T, topk, generator=g)
    wts = (wts / wts.sum(-1, keepdim=True)).numpy()
    got = oracle_mod.moe_ref(x, c13, s13, c2, s2, wts, ids)
    ac, as_ = oracle_mod.quant_mxfp8(x)
    out = np.zeros((T, H), np.float32)
    for t in range(T):
        for k in range(topk):
            e = ids[t, k]
            gu = oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(ac[t:t + 1], as_[t:t + 1], c13[e], s13[e], 2))
            mc, ms = oracle_mod.swiglu_mxfp8(gu)
            yk = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(mc, ms, c2[e], s2[e], 2)))
            out[t] = out[t] + yk[0] * np.float32(wts[t, k])
    assert np.array_equal(got, oracle_mod.f32_to_bf16(out))


def test_router_oracle_matches_torch_topk_softmax(oracle_mod):
    """Without ties the router oracle's ids are torch.topk of the softmax (the order vLLM's
    select_experts returns) and its weights the torch fp32 softmax / renormalization."""
    import torch
    g = torch.Generator().manual_seed(3)
    for T, E, k in [(7, 4, 2), (128, 256, 8), (33, 64, 6), (5, 1024, 16)]:
        logits = torch.randn(T, E, generator=g)
        for renorm in (True, False):
            w, ids, *_ = oracle_mod.moe_router(logits.numpy(), k, renorm)
            p = torch.softmax(logits.double(), -1)
            tw, tids = torch.topk(p, k, -1)
            if renorm:
                tw = tw / tw.sum(-1, keepdim=True)
            assert np.array_equal(ids, tids.int().numpy())
            np.testing.assert_allclose(w, tw.numpy(), rtol=1e-12, atol=0)


def test_router_oracle_ties_and_special_values(oracle_mod):
    """Ties go to the lower expert; -0 ties with +0; a brute-force restatement of the rule
    (repeatedly take the largest remaining value, lowest index first) agrees."""
    rng = np.random.default_rng(5)
    x = rng.integers(-3, 4, size=(64, 32)).astype(np.float32)  # many exact ties
    x[0, :4] = [0.0, -0.0, 0.0, -0.0]
    x[1, :] = 1.0
    for k in (1, 3, 8, 32):
        _, ids, *_ = oracle_mod.moe_router(x, k, True)
        for t in range(x.shape[0]):
            left = list(range(x.shape[1]))
            want = []
            for _ in range(k):
                best = max(left, key=lambda i: (x[t, i] + 0.0, -i))
                want.append(best)
                left.remove(best)
            assert list(ids[t]) == want, (t, k)
    _, ids, *_ = oracle_mod.moe_router(x[1:2], 4, True)
    assert list(ids[0]) == [0, 1, 2, 3]  # all equal: the lowest experts
    zeros = np.array([[-0.0, 0.0, -0.0, 0.0, -1.0]], np.float32)
    _, ids, *_ = oracle_mod.moe_router(zeros, 4, True)
    assert list(ids[0]) == [0, 1, 2, 3]  # -0 and +0 tie
    # renormalized weights are the selected probabilities rescaled to sum to one
    w, ids, *_ = oracle_mod.moe_router(x, 8, True)
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-12)
    w2, ids2, *_ = oracle_mod.moe_router(x, 8, False)
    assert np.array_equal(ids, ids2)
    np.testing.assert_allclose(w2 / w2.sum(1, keepdims=True), w, rtol=1e-12)


def test_router_oracle_sort_is_moe_route(oracle_mod):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((300, 64)).astype(np.float32)
    _, ids, s, o, inv = oracle_mod.moe_router(x, 4, True)
    rs, ro, rinv = oracle_mod.moe_route(ids, 64)
    assert np.array_equal(s, rs) and np.array_equal(o, ro) and np.array_equal(inv, rinv)
