"""GPU parity of the fused and grouped MoE schedules the reference's MoE API names
(_MOE_REQUIRED_API, src/vllm_mach/mxfp6/moe_utils.py:28-44; call sites
src/vllm_mach/mxfp6/moe.py:126-313): the small-batch sequence with a shared expert appended
(moe.py:398-426) against the layer run with the same routing through ``Mxfp6Experts``
(bit for bit) and the oracle's per-expert reference (the layer bar), and the grouped
sequence from router logits against ``Mxfp6Experts.apply_router``."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def api(pkg):
    from vllm_mach_amd import mxfp6_api
    mxfp6_api.load_library()
    return mxfp6_api


def _experts(oracle_mod, dev, E, H, I, seed, fmt=3):
    g = torch.Generator().manual_seed(seed)
    w13 = (torch.randn(E, 2 * I, H, generator=g) * 0.1).bfloat16()
    w2 = (torch.randn(E, H, I, generator=g) * 0.1).bfloat16()
    q13 = [oracle_mod.quant_mxfp6(w13[e], fmt) for e in range(E)]
    q2 = [oracle_mod.quant_mxfp6(w2[e], fmt) for e in range(E)]
    c13 = np.stack([c for c, _ in q13]); s13 = np.stack([s for _, s in q13])
    c2 = np.stack([c for c, _ in q2]); s2 = np.stack([s for _, s in q2])
    return c13, s13, c2, s2, g


@pytest.fixture(params=[False, True], ids=["combine-launch", "combine-in-w2"])
def fuse_combine(request, api, monkeypatch):
    monkeypatch.setattr(api, "FUSE_COMBINE", request.param)
    return request.param


@pytest.mark.parametrize("T", [1, 2, 4, 8])
def test_small_batch_schedule_with_shared_expert(pkg, api, oracle_mod, dev, T, fuse_combine):
    """router_quant -> w1 split-K SiLU -> w2 reduce (one token: qwen35_w2_splitk_reduce_out;
    more: array_gemm_w6a8_reduce_out), the shared expert as expert E with weight
    sigmoid(shared_gate)."""
    E, H, I, topk = 16, 256, 128, 4
    c13, s13, c2, s2, g = _experts(oracle_mod, dev, E + 1, H, I, 500 + T)
    w1 = torch.from_numpy(oracle_mod.pack_fp6(c13)).to(dev)
    w2 = torch.from_numpy(oracle_mod.pack_fp6(c2)).to(dev)
    s1 = api.pack_scales(torch.from_numpy(s13).to(dev))
    sw2 = api.pack_scales(torch.from_numpy(s2).to(dev))
    x = torch.randn(T, H, generator=g).bfloat16().to(dev)
    gate = (torch.randn(E + 1, H, generator=g) * 0.05).bfloat16().to(dev)
    routes = T * (topk + 1)
    quantized = torch.empty(T, H, dtype=torch.uint8, device=dev)
    in_scales = torch.empty(T, H // 32, dtype=torch.uint8, device=dev)
    logits = torch.empty(T, E, dtype=torch.bfloat16, device=dev)
    wts = torch.empty(T, topk, dtype=torch.float32, device=dev)
    ids = torch.empty(T, topk, dtype=torch.int32, device=dev)
    shared = torch.empty(T, dtype=torch.bfloat16, device=dev)
    api.qwen35_router_quant_out(quantized, in_scales, logits, wts, ids, shared, x, gate, renormalize=True)
    full = torch.matmul(x, gate.t())
    assert torch.equal(logits, full[:, :E]) and torch.equal(shared, full[:, E])
    rw, rids, *_ = oracle_mod.moe_router(logits.float().cpu().numpy(), topk, True)
    assert np.array_equal(ids.cpu().numpy(), rids)
    qc, qs = oracle_mod.quant_mxfp8(x.cpu(), oracle_mod.RULE_FLOOR_CARRY175)
    assert np.array_equal(quantized.cpu().numpy(), qc) and np.array_equal(in_scales.cpu().numpy(), qs)

    act = torch.empty(routes, I, dtype=torch.uint8, device=dev)
    act_s = torch.empty(routes, I // 32, dtype=torch.uint8, device=dev)
    api.qwen35_w1_splitk_silu_mxfp8_out(act, act_s, torch.empty(1, device=dev), quantized, in_scales, w1, s1, ids)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    if T == 1:
        api.qwen35_w2_splitk_reduce_out(out, torch.empty(1, device=dev), act, act_s, w2, sw2, ids, wts, shared)
    else:
        api.array_gemm_w6a8_reduce_out(out, act, act_s, w2, sw2, ids, wts, shared, use_packed_vector_loads=T == 4)

    # the same layer through Mxfp6Experts with the shared expert as the last route
    ids_ext = torch.cat([ids, torch.full((T, 1), E, dtype=torch.int32, device=dev)], 1)
    wts_ext = torch.cat([wts, torch.sigmoid(shared.float())[:, None]], 1)
    experts = pkg.Mxfp6Experts(fmt=3)
    e1, e2 = experts.process_weights_after_loading(w1, torch.from_numpy(s13).to(dev), w2,
                                                   torch.from_numpy(s2).to(dev))
    ref = torch.empty_like(out)
    experts.apply(ref, x, e1, e2, wts_ext, ids_ext, "silu", E + 1, None, None, None, None, None, None, False)
    assert torch.equal(out, ref)
    lay = oracle_mod.bf16_to_f32(oracle_mod.moe_ref(x.cpu(), c13, s13, c2, s2, wts_ext.cpu().numpy(),
                                                    ids_ext.cpu().numpy(), 3))
    got = out.float().cpu().numpy()
    assert np.linalg.norm(got - lay) / np.linalg.norm(lay) < 1e-2


@pytest.mark.parametrize("T,E,H,I,topk", [(7, 4, 256, 128, 2), (128, 256, 2048, 512, 8), (40, 16, 512, 256, 4)])
def test_grouped_schedule_from_logits(pkg, api, oracle_mod, dev, T, E, H, I, topk, fuse_combine):
    """qwen35_grouped_gemm_out + qwen35_grouped_reduce_out (moe.py:282-302) equal
    Mxfp6Experts.apply_router bit for bit; with a shared output, its addition in fp32
    before the one rounding; qwen35_grouped_moe_out from the same routing as well."""
    c13, s13, c2, s2, g = _experts(oracle_mod, dev, E, H, I, 900 + T)
    w1 = torch.from_numpy(oracle_mod.pack_fp6(c13)).to(dev)
    w2 = torch.from_numpy(oracle_mod.pack_fp6(c2)).to(dev)
    s1 = api.pack_scales(torch.from_numpy(s13).to(dev))
    sw2 = api.pack_scales(torch.from_numpy(s2).to(dev))
    x = torch.randn(T, H, generator=g).bfloat16().to(dev)
    logits = torch.randn(T, E, generator=g).to(dev)
    ws13, ws2 = api.qwen35_grouped_workspace_shapes(T, H, I, topk)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    work = api.Qwen35GroupedWorkspace.from_storage(out, torch.empty(ws13, dtype=torch.bfloat16, device=dev),
                                                   torch.empty(ws2, dtype=torch.bfloat16, device=dev))
    api.qwen35_grouped_gemm_out(work, x, logits, w1, s1, w2, sw2, renormalize=True)
    api.qwen35_grouped_reduce_out(work, out)
    experts = pkg.Mxfp6Experts(fmt=3)
    e1, e2 = experts.process_weights_after_loading(w1, torch.from_numpy(s13).to(dev), w2,
                                                   torch.from_numpy(s2).to(dev))
    ref = torch.empty_like(out)
    experts.apply_router(ref, x, e1, e2, logits, topk, True)
    assert torch.equal(out, ref)

    shared_out = torch.randn(T, H, generator=g).bfloat16().to(dev)
    out_s = torch.empty_like(out)
    api.qwen35_grouped_reduce_out(work, out_s, shared_out)
    y = oracle_mod.bf16_to_f32(oracle_mod.bf16_bits(work.workspace2.reshape(-1)[: T * topk * H].view(T * topk, H)))
    w = work.topk_weights.cpu().numpy().astype(np.float32)
    inv = work.inverse.cpu().numpy()
    acc = np.zeros((T, H), np.float32)
    for k in range(topk):  # route order, binary32, then the addend
        acc = acc + y[inv.reshape(T, topk)[:, k]] * w[:, k:k + 1]
    acc = acc + oracle_mod.bf16_to_f32(oracle_mod.bf16_bits(shared_out))
    assert np.array_equal(oracle_mod.bf16_bits(out_s), oracle_mod.f32_to_bf16(acc))

    out_m = torch.empty_like(out)
    api.qwen35_grouped_moe_out(work, out_m, x, w1, s1, w2, sw2, work.topk_weights, pkg.select_experts(logits, topk)[1])
    assert torch.equal(out_m, ref)
