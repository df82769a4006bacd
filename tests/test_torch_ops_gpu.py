"""GPU checks of torch.ops.dsa.*: each op equals the Python wrapper over the same C ABI
bit for bit, and a HIP-graph capture of quantiser -> indexer + top-k -> sparse MLA
replays to the eager results (several replays, eager work and host syncs between
them; the analogue of examples/aclgraph/ for these kernels)."""
import pytest
import torch

from oracle import dsa_oracle as ref

pytestmark = pytest.mark.gpu


def _pipeline_inputs(dev, seed=5):
    g = torch.Generator().manual_seed(seed)
    B, S, Skv, Hi, H, D, K = 1, 64, 2048, 64, 32, 128, 256
    return dict(
        qi=torch.randn(B * S * Hi, D, generator=g).to(torch.bfloat16).to(dev),
        ki=torch.randn(B * Skv, D, generator=g).to(torch.bfloat16).to(dev),
        w=(torch.randn(B, S, Hi, generator=g) / 8).to(dev),
        q=(torch.randn(B, S, H, 576, generator=g) * 0.5).to(torch.bfloat16).to(dev),
        kv=(torch.randn(B, Skv, 1, 576, generator=g) * 0.5).to(torch.bfloat16).to(dev),
        shape=(B, S, Skv, Hi, H, D, K))


def _pipeline(ops, t):
    B, S, Skv, Hi, H, D, K = t["shape"]
    q8, qs = ops.act_quant(t["qi"], False, torch.float8_e4m3fn)
    k8, ks = ops.act_quant(t["ki"], False, torch.float8_e4m3fn)
    w = t["w"] * qs.view(B, S, Hi)
    idx, _ = ops.lightning_indexer(q8.view(B, S, Hi, D), k8.view(B, Skv, 1, D), w, ks.view(B, Skv),
                                   sparse_count=K, sparse_mode=3)
    out, lse = ops.sparse_mla_fwd(t["q"], t["kv"], idx, 576 ** -0.5)
    return idx, out, lse


def test_ops_equal_python_wrappers(dsa, dev):
    ops = dsa.load_torch_ops()
    t = _pipeline_inputs(dev)
    B, S, Skv, Hi, H, D, K = t["shape"]
    y1, s1 = ops.act_quant(t["ki"], True, torch.int8)
    y2, s2 = dsa.act_quant(t["ki"], round_scale=True, dtype=torch.int8)
    assert torch.equal(y1, y2) and torch.equal(s1, s2)
    idx, out, lse = _pipeline(ops, t)
    q8, qs = dsa.act_quant(t["qi"], dtype=torch.float8_e4m3fn)
    k8, ks = dsa.act_quant(t["ki"], dtype=torch.float8_e4m3fn)
    idx2, _ = dsa.lightning_indexer(q8.view(B, S, Hi, D), k8.view(B, Skv, 1, D), t["w"], key_scale=ks.view(B, Skv),
                                    query_scale=qs.view(B, S, Hi), sparse_count=K, sparse_mode=3)
    assert torch.equal(idx, idx2)
    out2, lse2 = dsa.sparse_mla_fwd(t["q"], t["kv"], idx2, 576 ** -0.5)
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
    x = torch.randn(9, 40000, device=dev)
    i1, v1 = ops.topk_select(x, 512)
    i2, v2 = dsa.topk_selector(x, 512, sorted=True, return_values=True)
    ri, rv = ref.topk_stable(x.cpu(), 512)
    assert torch.equal(i1.cpu(), ri) and torch.equal(v1.cpu(), rv)
    assert torch.equal(i1, i2) and torch.equal(v1, v2)


def test_hip_graph_capture_and_replay(dsa, dev):
    ops = dsa.load_torch_ops()
    t = _pipeline_inputs(dev, seed=6)
    want = _pipeline(ops, t)                      # eager (also sets kernel attributes before capture)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _pipeline(ops, t)                         # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = _pipeline(ops, t)
    for rep in range(4):
        for o in got:
            o.zero_()                             # clobber the outputs between replays
        junk = torch.randn(1 << 20, device=dev).sum()  # unrelated eager work
        graph.replay()
        torch.cuda.synchronize()
        assert junk.isfinite()
        for a, b in zip(got, want):
            assert torch.equal(a, b), f"replay {rep}"
