"""GPU parity of the MoE path: token sort bit-exact, combine bit-exact, and the whole
routed-expert layer against the oracle's per-expert dense reference
(tests/native_mxfp6/test_moe.py:165-248: seed 12035, e=4, h=256, i=128, m=7, topk=2)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,topk,E", [(7, 2, 4), (1, 8, 256), (128, 8, 256), (2048, 8, 256), (3000, 4, 64)])
def test_route_bit_exact(pkg, oracle_mod, dev, T, topk, E):
    g = torch.Generator().manual_seed(T + E)
    logits = torch.randn(T, E, generator=g)
    ids = torch.topk(torch.softmax(logits, -1), topk, -1).indices.int()
    s, o, inv = torch.ops.mach_amd.moe_route(ids.to(dev), E)
    rs, ro, rinv = oracle_mod.moe_route(ids.numpy(), E)
    assert np.array_equal(o.cpu().numpy(), ro)
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(inv.cpu().numpy(), rinv)


def test_route_drops_out_of_range_ids(pkg, oracle_mod, dev):
    ids = torch.tensor([[0, 5], [-1, 1], [1, 0]], dtype=torch.int32)
    s, o, inv = torch.ops.mach_amd.moe_route(ids.to(dev), 2)
    rs, ro, rinv = oracle_mod.moe_route(ids.numpy(), 2)
    n = int(ro[-1])
    assert np.array_equal(o.cpu().numpy(), ro) and np.array_equal(inv.cpu().numpy(), rinv)
    assert np.array_equal(s.cpu().numpy()[:n], rs[:n])


@pytest.mark.parametrize("T,topk,H", [(7, 2, 256), (2048, 8, 2048)])
def test_reduce_bit_exact(pkg, oracle_mod, dev, T, topk, H):
    g = torch.Generator().manual_seed(12035)
    y = torch.randn(T * topk, H, generator=g).bfloat16()
    w = torch.rand(T, topk, generator=g)
    w /= w.sum(-1, keepdim=True)
    inverse = torch.randperm(T * topk, generator=g).int()
    inverse[0] = -1  # a dropped route
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    torch.ops.mach_amd.moe_reduce(out, y.to(dev), w.to(dev), inverse.to(dev))
    ref = oracle_mod.moe_reduce(oracle_mod.bf16_bits(y), w.numpy(), inverse.numpy())
    assert np.array_equal(oracle_mod.bf16_bits(out), ref)


def _moe_case(oracle_mod, E, H, I, T, topk, seed, fmt=2, std=0.1):
    g = torch.Generator().manual_seed(seed)
    w13 = (torch.randn(E, 2 * I, H, generator=g) * std).bfloat16()
    w2 = (torch.randn(E, H, I, generator=g) * std).bfloat16()
    q13 = [oracle_mod.quant_mxfp6(w13[e], fmt) for e in range(E)]
    q2 = [oracle_mod.quant_mxfp6(w2[e], fmt) for e in range(E)]
    c13 = np.stack([c for c, _ in q13]); s13 = np.stack([s for _, s in q13])
    c2 = np.stack([c for c, _ in q2]); s2 = np.stack([s for _, s in q2])
    x = torch.randn(T, H, generator=g).bfloat16()
    logits = torch.randn(T, E, generator=g)
    wts, ids = torch.topk(torch.softmax(logits, -1), topk, -1)
    wts = (wts / wts.sum(-1, keepdim=True)).float()
    return c13, s13, c2, s2, x, wts, ids.int()


@pytest.mark.parametrize("E,H,I,T,topk,fmt", [
    (4, 256, 128, 7, 2, 2),
    (4, 256, 128, 7, 2, 3),
    (32, 2048, 512, 128, 8, 2),
])
def test_moe_layer_matches_oracle(pkg, oracle_mod, dev, E, H, I, T, topk, fmt):
    c13, s13, c2, s2, x, wts, ids = _moe_case(oracle_mod, E, H, I, T, topk, 12035, fmt)
    experts = pkg.Mxfp6Experts(fmt=fmt)
    w1, w2 = experts.process_weights_after_loading(
        torch.from_numpy(oracle_mod.pack_fp6(c13)).to(dev), torch.from_numpy(s13).to(dev),
        torch.from_numpy(oracle_mod.pack_fp6(c2)).to(dev), torch.from_numpy(s2).to(dev))
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    experts.apply(out, x.to(dev), w1, w2, wts.to(dev), ids.to(dev), "silu", E, None,
                  None, None, None, None, None, False)
    ref = oracle_mod.bf16_to_f32(oracle_mod.moe_ref(x, c13, s13, c2, s2, wts.numpy(), ids.numpy(), fmt))
    got = out.float().cpu().numpy()
    # the reference's tolerance (test_moe.py:248) and the relative Frobenius bar
    np.testing.assert_allclose(got, ref, rtol=0.03, atol=0.03)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel < 1e-2, rel


def test_moe_graph_replay_changing_routes(pkg, oracle_mod, dev):
    """Captured layer replayed with new hidden states and rotated expert ids
    (tests/native_mxfp6/test_moe.py:216-248)."""
    E, H, I, T, topk = 4, 256, 128, 7, 2
    c13, s13, c2, s2, x, wts, ids = _moe_case(oracle_mod, E, H, I, T, topk, 12035)
    experts = pkg.Mxfp6Experts(fmt=2)
    w1, w2 = experts.process_weights_after_loading(
        torch.from_numpy(oracle_mod.pack_fp6(c13)).to(dev), torch.from_numpy(s13).to(dev),
        torch.from_numpy(oracle_mod.pack_fp6(c2)).to(dev), torch.from_numpy(s2).to(dev))
    xd, wd, idd = x.to(dev), wts.to(dev), ids.to(dev)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)

    def run():
        experts.apply(out, xd, w1, w2, wd, idd, "silu", E, None, None, None, None, None, None, False)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        run()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            run()
        for shift in range(3):
            xd.normal_()
            idd.copy_(torch.tensor([[(j + shift) % E, (j + shift + 1) % E] for j in range(T)], dtype=torch.int32))
            graph.replay()
            stream.synchronize()
            ref = oracle_mod.moe_ref(xd.cpu(), c13, s13, c2, s2, wd.cpu().numpy(), idd.cpu().numpy(), 2)
            np.testing.assert_allclose(out.float().cpu().numpy(), oracle_mod.bf16_to_f32(ref), rtol=0.03, atol=0.03)
    torch.cuda.current_stream().wait_stream(stream)
