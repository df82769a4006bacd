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


def test_hip_graph_capture_decode_shapes(dsa, dev):
    # Decode-shaped calls in one graph: the key-split indexer (2 query rows), the decode
    # kernel in 128-slot chunks with its combine (sparse MLA, 576-wide, topk 512) and in
    # one workgroup per row (sparse_attn, topk 200); replays equal the eager results.
    ops = dsa.load_torch_ops()
    g = torch.Generator().manual_seed(8)
    B, S, Skv, Hi, H, D, K = 1, 2, 2048, 64, 32, 128, 512
    t = dict(qi=torch.randn(B * S * Hi, D, generator=g).to(torch.bfloat16).to(dev),
             ki=torch.randn(B * Skv, D, generator=g).to(torch.bfloat16).to(dev),
             w=(torch.randn(B, S, Hi, generator=g) / 8).to(dev),
             q=(torch.randn(B, S, H, 576, generator=g) * 0.5).to(torch.bfloat16).to(dev),
             kv=(torch.randn(B, Skv, 1, 576, generator=g) * 0.5).to(torch.bfloat16).to(dev),
             shape=(B, S, Skv, Hi, H, D, K))
    qa = (torch.randn(2, 3, 16, 512, generator=g)).to(torch.bfloat16).to(dev)
    kva = (torch.randn(2, 300, 512, generator=g)).to(torch.bfloat16).to(dev)
    sink = torch.randn(16, generator=g).to(dev)
    ia = torch.randint(0, 300, (2, 3, 200), generator=g, dtype=torch.int32).to(dev)

    def run():
        a = ops.sparse_attn(qa, kva, sink, ia, 0.05)
        return _pipeline(ops, t) + (tuple(a) if isinstance(a, (tuple, list)) else (a,))

    want = run()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = run()
    for rep in range(3):
        for o in got:
            o.zero_()
        junk = torch.randn(1 << 20, device=dev).sum()
        graph.replay()
        torch.cuda.synchronize()
        assert junk.isfinite()
        for a, b in zip(got, want):
            assert torch.equal(a, b), f"replay {rep}"


def _raises(fn, match):
    with pytest.raises(RuntimeError, match=match):
        fn()


def test_ops_reject_host_and_misshaped_arguments(dsa, dev):
    """Every tensor argument of every op is checked before a kernel is launched: a host tensor
    (the torch_npu convention for sequence lengths) or a short buffer raises."""
    ops = dsa.load_torch_ops()
    g = torch.Generator().manual_seed(9)
    B, S, Skv, H, Hi, D = 2, 4, 256, 16, 16, 128
    qi = torch.randn(B, S, Hi, D, generator=g).to(torch.bfloat16).to(dev)
    ki = torch.randn(B, Skv, 1, D, generator=g).to(torch.bfloat16).to(dev)
    w = torch.randn(B, S, Hi, generator=g).to(dev)
    lens = torch.tensor([S, S], dtype=torch.int32)
    ops.lightning_indexer(qi, ki, w, sparse_count=16)                      # well-formed: runs
    _raises(lambda: ops.lightning_indexer(qi, ki, w, actual_seq_lengths_query=lens), "must be on")
    _raises(lambda: ops.lightning_indexer(qi, ki, w, actual_seq_lengths_key=lens[:1].to(dev)), "elements")
    _raises(lambda: ops.lightning_indexer(qi, ki, w[:, :2]), "weights")
    _raises(lambda: ops.lightning_indexer(qi, ki, w, torch.ones(B * Skv)), "key_scale")
    _raises(lambda: ops.lightning_indexer(qi, ki, w, torch.ones(B, Skv - 1, device=dev)), "key_scale")
    _raises(lambda: ops.lightning_indexer(qi, ki[:1], w), "batch")
    _raises(lambda: ops.lightning_indexer(qi, ki, w, block_table=torch.zeros(B, 4, dtype=torch.int32)),
            "must be on|s2")
    q = torch.randn(B, S, H, 576, generator=g).to(torch.bfloat16).to(dev)
    kv = torch.randn(B, Skv, 1, 576, generator=g).to(torch.bfloat16).to(dev)
    idx = torch.randint(0, 64, (B, S, 1, 32), generator=g, dtype=torch.int32).to(dev)
    sm = 576 ** -0.5
    _raises(lambda: ops.sparse_mla_fwd(q, kv, idx, sm, actual_seq_lengths_kv=lens), "must be on")
    _raises(lambda: ops.sparse_mla_fwd(q, kv, idx, sm, block_table=torch.zeros(B, 4, dtype=torch.int32)),
            "must be on")
    _raises(lambda: ops.sparse_mla_fwd(q, kv, idx, sm, block_table=torch.zeros(1, 4, dtype=torch.int32,
                                                                                 device=dev)), "block_table")
    _raises(lambda: ops.sparse_mla_fwd(q[..., :512].contiguous(), kv, idx, sm), "576")
    _raises(lambda: ops.sparse_mla_fwd(q, kv[..., :512].contiguous(), idx, sm), "576")
    _raises(lambda: ops.sparse_mla_fwd(q, kv, idx[:, :2].contiguous(), sm), "indices")
    _raises(lambda: ops.sparse_mla_fwd(q, kv[:1], idx, sm), "batch")
    qa = torch.randn(1, 3, 16, 512, generator=g).to(torch.bfloat16).to(dev)
    kva = torch.randn(1, 40, 512, generator=g).to(torch.bfloat16).to(dev)
    ia = torch.randint(0, 40, (1, 3, 8), generator=g, dtype=torch.int32).to(dev)
    ops.sparse_attn(qa, kva, torch.zeros(16, device=dev), ia, 0.04)     # well-formed: runs
    _raises(lambda: ops.sparse_attn(qa, kva, torch.zeros(16), ia, 0.04), "must be on")
    _raises(lambda: ops.sparse_attn(qa, kva, torch.zeros(8, device=dev), ia, 0.04), "attn_sink")
    _raises(lambda: ops.sparse_attn(qa, kva, None, ia.cpu(), 0.04), "must be on")
    _raises(lambda: ops.sparse_attn(qa, kva, None, ia[:, :2].contiguous(), 0.04), "topk_idxs")
    T, bs = 5, 128
    qv = torch.randn(T, 16, 512, generator=g).to(torch.bfloat16).to(dev)
    cache = torch.randn(4, bs, 1, 512, generator=g).to(torch.bfloat16).to(dev)
    bt = torch.arange(4, dtype=torch.int32, device=dev).view(1, 4)
    qs = torch.tensor([0], dtype=torch.int32, device=dev)
    ql = torch.tensor([T], dtype=torch.int32, device=dev)
    kl = torch.tensor([300], dtype=torch.int32, device=dev)
    sinks = torch.zeros(16, device=dev)
    ops.sparse_flash_mla(qv, cache, bt, qs, ql, kl, sinks, 0.04)         # well-formed: runs
    _raises(lambda: ops.sparse_flash_mla(qv, cache, bt, qs.cpu(), ql, kl, sinks, 0.04), "must be on")
    _raises(lambda: ops.sparse_flash_mla(qv, cache, bt, qs, ql, kl.cpu(), sinks, 0.04), "must be on")
    _raises(lambda: ops.sparse_flash_mla(qv, cache, bt, qs, ql, kl, sinks.cpu(), 0.04), "must be on")
    _raises(lambda: ops.sparse_flash_mla(qv, cache, bt, qs, ql, kl, sinks[:8], 0.04), "sinks")
    _raises(lambda: ops.sparse_flash_mla(qv, cache, bt.cpu(), qs, ql, kl, sinks, 0.04), "must be on")
    _raises(lambda: ops.sparse_flash_mla(qv, cache, bt, qs, ql, kl, sinks, 0.04, cache, bt), "max_cmp")
    _raises(lambda: ops.sparse_flash_mla(qv, cache, bt, qs, ql, kl, sinks, 0.04, cache, None,
                                         torch.zeros(T, 8, dtype=torch.int32, device=dev)), "cmp_block_table")
    _raises(lambda: ops.sparse_flash_mla(qv, cache, bt, qs, ql, kl, sinks, 0.04, cache, bt,
                                         torch.zeros(T - 1, 8, dtype=torch.int32, device=dev)), "cmp_sparse_indices")
    torch.cuda.synchronize()


def test_op_hca_matches_python_wrapper(dsa, dev):
    """sparse_flash_mla in "hca" mode (compressed rows without selection lists) through the op,
    with max_cmp = seqused_kv.max() // cmp_ratio as the reference API derives it, equals the
    Python wrapper bit for bit."""
    ops = dsa.load_torch_ops()
    g = torch.Generator().manual_seed(12)
    H, bs, ratio, win = 64, 128, 4, 127
    kv_len = [700, 1500]
    q_len = [3, 5]
    T = sum(q_len)
    ob = [(n + bs - 1) // bs for n in kv_len]
    cb = [((n // ratio) + bs - 1) // bs for n in kv_len]
    q = torch.randn(T, H, 512, generator=g).to(torch.bfloat16).to(dev)
    ori = torch.randn(sum(ob), bs, 1, 512, generator=g).to(torch.bfloat16).to(dev)
    cmp = torch.randn(sum(cb), bs, 1, 512, generator=g).to(torch.bfloat16).to(dev)
    obt = torch.full((2, max(ob)), -1, dtype=torch.int32)
    cbt = torch.full((2, max(cb)), -1, dtype=torch.int32)
    obt[0, :ob[0]] = torch.arange(ob[0])
    obt[1, :ob[1]] = torch.arange(ob[0], ob[0] + ob[1])
    cbt[0, :cb[0]] = torch.arange(cb[0])
    cbt[1, :cb[1]] = torch.arange(cb[0], cb[0] + cb[1])
    obt, cbt = obt.to(dev), cbt.to(dev)
    qs = torch.tensor([0, q_len[0]], dtype=torch.int32, device=dev)
    ql = torch.tensor(q_len, dtype=torch.int32, device=dev)
    kl = torch.tensor(kv_len, dtype=torch.int32, device=dev)
    sinks = torch.randn(H, generator=g).to(dev)
    scale = 512 ** -0.5
    o1, l1 = ops.sparse_flash_mla(q, ori, obt, qs, ql, kl, sinks, scale, cmp, cbt, None, ratio, win,
                                  max(kv_len) // ratio)
    cu = torch.tensor([0] + list(torch.tensor(q_len).cumsum(0)), dtype=torch.int32, device=dev)
    o2, l2 = dsa.sparse_flash_mla(q, ori_kv=ori, cmp_kv=cmp, ori_block_table=obt, cmp_block_table=cbt,
                                  cu_seqlens_q=cu, seqused_kv=kl, sinks=sinks, softmax_scale=scale,
                                  cmp_ratio=ratio, ori_mask_mode=4, cmp_mask_mode=3, ori_win_left=win,
                                  ori_win_right=0, layout_q="TND", layout_kv="PA_ND",
                                  return_softmax_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2.view_as(o1)) and torch.equal(l1, l2.view_as(l1))
