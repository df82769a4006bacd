"""GPU parity of the fused (streaming) indexer -> top-k against the dense path and the oracle.

The fused entry (``dsa_lightning_indexer_fused``) must give the dense path's
output bit for bit: the same indices (sorted by score desc, index asc, -1
padded) and the same values, on every path it can take -- the streamed top-k,
rows with at most k valid keys (no threshold), and rows sent back to the dense
logits because the sampled threshold was too high, a key chunk overflowed its
candidate slot, or ties defeated the register top-k.  Inputs that force each
fallback are built from the data (key scales), not from switches in the code.
"""
import pytest
import torch

from oracle import dsa_oracle as ref

pytestmark = pytest.mark.gpu


def _inputs(B, S1, S2, H, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    qf = torch.randn(B, S1, H, D, generator=g)
    kf = torch.randn(B, S2, D, generator=g)
    w = torch.randn(B, S1, H, generator=g) / 8
    if dtype == torch.float8_e4m3fn:
        q = qf.to(torch.float8_e4m3fn)
        k, ks = ref.fp8_quantize_per_token(kf)
    else:
        q, k, ks = qf.to(dtype), kf.to(dtype), torch.ones(B, S2)
    return q, k, w, ks


def _both(dsa, dev, q, k, w, ks, K, **kw):
    args = (q.to(dev), k.to(dev), w.to(dev))
    kw = dict(kw, key_scale=ks.to(dev), sparse_count=K)
    a = dsa.lightning_indexer(*args, fuse_topk=True, **kw)
    b = dsa.lightning_indexer(*args, fuse_topk=False, **kw)
    torch.cuda.synchronize()
    return a, b


def _fused_c(dsa, dev, q, k, w, ks, K):
    """The fused entry through the C ABI (contiguous BSND keys): (indices, values, rows sent
    back to dense logits by a too-high threshold or a chunk overflow)."""
    lib = dsa.load_library()
    B, S1, H, D = q.shape
    S2 = k.shape[1]
    qd, kd, wd, ksd = q.to(dev), k.contiguous().to(dev), w.float().to(dev), ks.float().to(dev)
    idx = torch.empty((B, S1, K), dtype=torch.int32, device=dev)
    val = torch.empty((B, S1, K), dtype=torch.float32, device=dev)
    nb = lib.dsa_lightning_indexer_fused_workspace_size(B, S1, S2, K)
    ws = torch.empty((nb,), dtype=torch.uint8, device=dev)
    cnt = torch.full((1,), -1, dtype=torch.int32, device=dev)
    kind = 0 if q.dtype == torch.float8_e4m3fn else 1
    st = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.dsa_lightning_indexer_fused(kind, qd.data_ptr(), kd.data_ptr(), ksd.data_ptr(), wd.data_ptr(), B, S1,
                                         S2, H, D, None, None, None, 0, 0, 3, K, idx.data_ptr(), val.data_ptr(),
                                         ws.data_ptr(), nb, st)
    assert rc == 0
    assert lib.dsa_lightning_indexer_fused_fallback_rows(ws.data_ptr(), B, S1, S2, K, cnt.data_ptr(), st) == 0
    torch.cuda.synchronize()
    return idx.view(B, S1, 1, K), val.view(B, S1, 1, K), int(cnt.item())


def _applies(dsa, B, S1, S2, K):
    return dsa.load_library().dsa_lightning_indexer_fused_applies(B, S1, S2, K) == 1


@pytest.mark.parametrize("sparse_mode", [3, 0])
def test_fused_equals_dense_c2_shape(dsa, dev, sparse_mode):
    """C2's row length (32768 keys, 64 fp8 heads, top-2048) on 256 query rows at the tail."""
    B, S1, S2, H, D, K = 1, 256, 32768, 64, 128, 2048
    print(f"fused indexer C2 shape mode={sparse_mode}", flush=True)
    assert _applies(dsa, B, S1, S2, K)
    q, k, w, ks = _inputs(B, S1, S2, H, D, torch.float8_e4m3fn, 31)
    (fi, fv), (di, dv) = _both(dsa, dev, q, k.unsqueeze(2), w, ks, K, sparse_mode=sparse_mode, return_value=True)
    assert torch.equal(fi, di) and torch.equal(fv, dv)
    if sparse_mode == 3:  # the streamed path did the work: no row went back to dense logits
        ci, cv, nfb = _fused_c(dsa, dev, q, k, w, ks, K)
        assert nfb == 0 and torch.equal(ci, di) and torch.equal(cv, dv)
    # Anchored on the oracle too: its top-k of the GPU logits, on every row.
    logits = dsa.indexer_logits(q.to(dev), k.unsqueeze(2).to(dev), w.to(dev), ks.to(dev),
                                sparse_mode=sparse_mode).cpu().view(S1, S2)
    ri, rv = ref.topk_stable(logits, K)
    assert torch.equal(fi.cpu().view(S1, K), ri) and torch.equal(fv.cpu().view(S1, K), rv)


def test_fused_ragged_bf16_short_rows(dsa, dev):
    """bf16, D 64, 32 heads, two batches with actual lengths: rows with fewer valid keys than k
    (no threshold), rows just above k, padded query rows; S2 not a multiple of 64."""
    B, S1, S2, H, D, K = 2, 96, 20000, 32, 64, 1024
    print("fused indexer ragged bf16", flush=True)
    assert _applies(dsa, B, S1, S2, K)
    q, k, w, ks = _inputs(B, S1, S2, H, D, torch.bfloat16, 32)
    aq = torch.tensor([96, 40], dtype=torch.int32)
    ak = torch.tensor([20000, 1100], dtype=torch.int32)
    (fi, fv), (di, dv) = _both(dsa, dev, q, k.unsqueeze(2), w, ks, K, sparse_mode=3, return_value=True,
                               actual_seq_lengths_query=aq.to(dev), actual_seq_lengths_key=ak.to(dev))
    assert torch.equal(fi, di) and torch.equal(fv.float(), dv.float())
    assert (fi[1, :40] >= 0).sum(-1).max().item() <= 1100 and (fi[1, 40:] == -1).all()


def test_fused_paged_keys(dsa, dev):
    B, S1, S2, H, D, K, bs = 2, 48, 16384, 64, 128, 2048, 64
    print("fused indexer paged", flush=True)
    q, k, w, ks = _inputs(B, S1, S2, H, D, torch.float8_e4m3fn, 33)
    nblk = S2 // bs
    perm = torch.randperm(B * nblk, generator=torch.Generator().manual_seed(4))
    table = perm.view(B, nblk).to(torch.int32)
    pool = torch.empty(B * nblk, bs, 1, D, dtype=torch.float8_e4m3fn)
    pscale = torch.empty(B * nblk, bs)
    for b in range(B):
        pool[table[b].long()] = k[b].view(nblk, bs, 1, D)
        pscale[table[b].long()] = ks[b].view(nblk, bs)
    ak = torch.tensor([16384, 9000], dtype=torch.int32)
    (fi, _), (di, _) = _both(dsa, dev, q, pool, w, pscale, K, block_table=table.to(dev), layout_key="PA_BSND",
                             actual_seq_lengths_key=ak.to(dev))
    assert torch.equal(fi, di)
    # The paged call equals the contiguous one.
    ci, _ = dsa.lightning_indexer(q.to(dev), k.unsqueeze(2).to(dev), w.to(dev), key_scale=ks.to(dev),
                                  sparse_count=K, actual_seq_lengths_key=ak.to(dev), fuse_topk=True)
    assert torch.equal(fi, ci)


def test_fused_threshold_too_high_falls_back(dsa, dev):
    """Sampled keys (the first 64 of every 1024 at S2 = 32768) scaled up 50x: the sampled
    threshold sits above every other key, fewer than k keys reach it, every row is recomputed
    densely."""
    B, S1, S2, H, D, K = 1, 64, 32768, 64, 128, 2048
    print("fused indexer forced fallback (threshold)", flush=True)
    q, k, w, ks = _inputs(B, S1, S2, H, D, torch.float8_e4m3fn, 34)
    pos = torch.arange(S2)
    ks = torch.where((pos % 1024) < 64, ks * 50, ks)
    (fi, fv), (di, dv) = _both(dsa, dev, q, k.unsqueeze(2), w, ks, K, return_value=True)
    assert torch.equal(fi, di) and torch.equal(fv, dv)
    ci, cv, nfb = _fused_c(dsa, dev, q, k, w, ks, K)
    assert nfb == S1 and torch.equal(ci, di) and torch.equal(cv, dv)


def test_fused_chunk_overflow_falls_back(dsa, dev):
    """k = 256: each key chunk keeps at most 2 k + 1024 = 1536 keys; the first chunk's unsampled
    keys scaled up 50x (3840 of them) overflow it."""
    B, S1, S2, H, D, K = 1, 64, 32768, 64, 128, 256
    print("fused indexer forced fallback (overflow)", flush=True)
    q, k, w, ks = _inputs(B, S1, S2, H, D, torch.float8_e4m3fn, 35)
    pos = torch.arange(S2)
    ks = torch.where((pos < 4096) & ((pos % 1024) >= 64), ks * 50, ks)
    (fi, fv), (di, dv) = _both(dsa, dev, q, k.unsqueeze(2), w, ks, K, return_value=True)
    assert torch.equal(fi, di) and torch.equal(fv, dv)
    ci, cv, nfb = _fused_c(dsa, dev, q, k, w, ks, K)
    assert nfb > 0 and torch.equal(ci, di) and torch.equal(cv, dv)


def test_fused_fallback_in_several_rounds(dsa, dev):
    """Rows sent back to the dense logits (sampled keys scaled up 50x), more of them than the
    bounded fallback buffer holds: 600 rows of 65536 keys go back in three rounds of 256."""
    B, S1, S2, H, D, K = 1, 600, 65536, 64, 128, 512
    print("fused indexer fallback rounds", flush=True)
    assert _applies(dsa, B, S1, S2, K)
    q, k, w, ks = _inputs(B, S1, S2, H, D, torch.float8_e4m3fn, 38)
    pos = torch.arange(S2)
    ks = torch.where((pos % 1024) < 64, ks * 50, ks)  # covers every sampled tile (64 of each 2048)
    ci, cv, nfb = _fused_c(dsa, dev, q, k, w, ks, K)
    (fi, fv), (di, dv) = _both(dsa, dev, q, k.unsqueeze(2), w, ks, K, return_value=True)
    assert nfb >= S1 * 9 // 10  # rows in every round
    assert torch.equal(fi, di) and torch.equal(fv, dv)
    assert torch.equal(ci, di) and torch.equal(cv, dv)


@pytest.mark.parametrize("K", [8192, 6144])
def test_fused_large_k_radix_path(dsa, dev, K):
    """sparse_count 6144 and 8192 (the reference's largest): the candidates of every row are
    packed and ranked by the exact radix kernel; equal to the dense path bit for bit."""
    B, S1, S2, H, D = 1, 192, 65536, 64, 128
    print(f"fused indexer k={K}", flush=True)
    assert _applies(dsa, B, S1, S2, K)
    q, k, w, ks = _inputs(B, S1, S2, H, D, torch.float8_e4m3fn, 39)
    ci, cv, nfb = _fused_c(dsa, dev, q, k, w, ks, K)
    di, dv = dsa.lightning_indexer(q.to(dev), k.unsqueeze(2).to(dev), w.to(dev), key_scale=ks.to(dev),
                                   sparse_count=K, return_value=True, fuse_topk=False)
    torch.cuda.synchronize()
    assert nfb == 0
    assert torch.equal(ci, di) and torch.equal(cv, dv)
    # And with every row forced back to the dense logits.
    pos = torch.arange(S2)
    ks2 = torch.where((pos % 1024) < 64, ks * 50, ks)
    ci2, cv2, nfb2 = _fused_c(dsa, dev, q, k, w, ks2, K)
    di2, dv2 = dsa.lightning_indexer(q.to(dev), k.unsqueeze(2).to(dev), w.to(dev), key_scale=ks2.to(dev),
                                     sparse_count=K, return_value=True, fuse_topk=False)
    torch.cuda.synchronize()
    # Most rows go back (a row whose scaled samples are mostly negative gets a low threshold
    # and keeps its top k in the stream).
    assert nfb2 >= S1 * 9 // 10 and torch.equal(ci2, di2) and torch.equal(cv2, dv2)


def test_fused_heavy_ties(dsa, dev):
    """Most key scales zero: most logits are exactly 0, ties everywhere (lower index wins)."""
    B, S1, S2, H, D, K = 1, 64, 32768, 64, 128, 2048
    print("fused indexer ties", flush=True)
    q, k, w, ks = _inputs(B, S1, S2, H, D, torch.float8_e4m3fn, 36)
    ks = torch.where(torch.arange(S2) % 7 == 0, ks, torch.zeros_like(ks))
    (fi, fv), (di, dv) = _both(dsa, dev, q, k.unsqueeze(2), w, ks, K, return_value=True)
    assert torch.equal(fi, di) and torch.equal(fv, dv)


def test_fused_long_rows_two_stage_shape(dsa, dev):
    """S2 = 65536 (the dense path takes the two-stage top-k there), 32 rows at the tail."""
    B, S1, S2, H, D, K = 1, 32, 65536, 64, 128, 2048
    print("fused indexer long rows", flush=True)
    q, k, w, ks = _inputs(B, S1, S2, H, D, torch.float8_e4m3fn, 37)
    (fi, fv), (di, dv) = _both(dsa, dev, q, k.unsqueeze(2), w, ks, K, return_value=True)
    assert torch.equal(fi, di) and torch.equal(fv, dv)


def test_fused_entry_on_a_short_shape_runs_dense(dsa, dev):
    B, S1, S2, H, D, K = 1, 16, 4096, 64, 128, 2048
    assert not _applies(dsa, B, S1, S2, K)
    q, k, w, ks = _inputs(B, S1, S2, H, D, torch.float8_e4m3fn, 38)
    (fi, _), (di, _) = _both(dsa, dev, q, k.unsqueeze(2), w, ks, K)
    assert torch.equal(fi, di)


def test_fused_tied_candidates_resolved_on_packed_rows(dsa, dev):
    """700 copies of one key (same row, same scale, x3) at unsampled positions: where their logit
    is large they all become candidates with one value -- a bin the register top-k will not rank,
    resolved by the exact kernel on the packed candidates (no dense recompute)."""
    B, S1, S2, H, D, K = 1, 64, 32768, 64, 128, 2048
    print("fused indexer tied candidates", flush=True)
    q, k, w, ks = _inputs(B, S1, S2, H, D, torch.float8_e4m3fn, 39)
    pos = torch.arange(S2)
    clones = pos[(pos % 1024) >= 64][::40][:700]
    k = k.clone()
    k[0, clones] = k[0, 5].clone()
    ks = ks.clone()
    ks[0, clones] = ks[0, 5] * 3
    (fi, fv), (di, dv) = _both(dsa, dev, q, k.unsqueeze(2), w, ks, K, return_value=True)
    assert torch.equal(fi, di) and torch.equal(fv, dv)
    ci, cv, nfb = _fused_c(dsa, dev, q, k, w, ks, K)
    assert nfb == 0 and torch.equal(ci, di) and torch.equal(cv, dv)


def test_fused_default_torch_op_and_graph_capture(dsa, dev):
    """2048 rows over 32768 keys take the fused path by default, in the wrapper and in
    torch.ops.dsa.lightning_indexer; the op captured in a HIP graph replays to the same output."""
    B, S1, S2, H, D, K = 1, 2048, 40960, 64, 128, 2048
    print("fused indexer default path + graph", flush=True)
    q, k, w, ks = _inputs(B, S1, S2, H, D, torch.float8_e4m3fn, 40)
    qd, kd, wd, ksd = q.to(dev), k.unsqueeze(2).to(dev), w.to(dev), ks.to(dev)
    di, dv = dsa.lightning_indexer(qd, kd, wd, key_scale=ksd, sparse_count=K, return_value=True, fuse_topk=False)
    ai, av = dsa.lightning_indexer(qd, kd, wd, key_scale=ksd, sparse_count=K, return_value=True)
    ops = dsa.load_torch_ops()
    oi, ov = ops.lightning_indexer(qd, kd, wd, ksd, sparse_count=K, sparse_mode=3, return_value=True)
    torch.cuda.synchronize()
    assert torch.equal(ai, di) and torch.equal(av, dv) and torch.equal(oi, di) and torch.equal(ov, dv)
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        ops.lightning_indexer(qd, kd, wd, ksd, sparse_count=K, sparse_mode=3, return_value=True)
    torch.cuda.current_stream(dev).wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gi, gv = ops.lightning_indexer(qd, kd, wd, ksd, sparse_count=K, sparse_mode=3, return_value=True)
    for _ in range(3):
        gi.fill_(7)
        gv.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gi, di) and torch.equal(gv, dv)


@pytest.mark.parametrize("case", range(6))
def test_fused_random_shapes(dsa, dev, case):
    """Seeded random shapes: batch 1-3, 8-160 query rows, 16384-70000 keys, k in {1, 77, 1000, 2048,
    4096}, ragged lengths, causal or full, fp8 / bf16 / fp16, 16-64 heads; bit-equal to the dense path."""
    g = torch.Generator().manual_seed(1000 + case)
    r = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=g))
    B, S1 = r(1, 3), r(8, 160)
    K = [1, 77, 1000, 2048, 4096][r(0, 4)]
    S2 = max(r(16384, 70000), 8 * K)
    H = [16, 32, 64][r(0, 2)]
    dtype = [torch.float8_e4m3fn, torch.bfloat16, torch.float16][case % 3]
    D = 128 if dtype == torch.float8_e4m3fn else 64
    mode = [3, 0][r(0, 1)]
    print(f"fused random case {case}: B={B} S1={S1} S2={S2} K={K} H={H} D={D} {dtype} mode={mode}", flush=True)
    assert _applies(dsa, B, S1, S2, K)
    q, k, w, ks = _inputs(B, S1, S2, H, D, dtype, 2000 + case)
    aq = torch.tensor([r(1, S1) for _ in range(B)], dtype=torch.int32)
    ak = torch.tensor([r(1, S2) for _ in range(B)], dtype=torch.int32)
    (fi, fv), (di, dv) = _both(dsa, dev, q, k.unsqueeze(2), w, ks, K, sparse_mode=mode, return_value=True,
                               actual_seq_lengths_query=aq.to(dev), actual_seq_lengths_key=ak.to(dev))
    assert torch.equal(fi, di) and torch.equal(fv.float(), dv.float())


def test_fused_fallback_under_graph_replay(dsa, dev):
    """The fused entry captured in a HIP graph on inputs that send every row back to the dense path
    (sampled keys scaled up), replayed with the outputs clobbered in between: every replay equals the
    dense path, and no flag or packed length from one replay leaks into the next."""
    B, S1, S2, H, D, K = 1, 64, 32768, 64, 128, 2048
    print("fused indexer fallback under graph replay", flush=True)
    q, k, w, ks = _inputs(B, S1, S2, H, D, torch.float8_e4m3fn, 41)
    pos = torch.arange(S2)
    ks = torch.where((pos % 1024) < 64, ks * 50, ks)
    di, dv = dsa.lightning_indexer(q.to(dev), k.unsqueeze(2).to(dev), w.to(dev), key_scale=ks.to(dev),
                                   sparse_count=K, return_value=True, fuse_topk=False)
    lib = dsa.load_library()
    qd, kd, wd, ksd = q.to(dev), k.contiguous().to(dev), w.float().to(dev), ks.float().to(dev)
    idx = torch.empty((B, S1, K), dtype=torch.int32, device=dev)
    val = torch.empty((B, S1, K), dtype=torch.float32, device=dev)
    nb = lib.dsa_lightning_indexer_fused_workspace_size(B, S1, S2, K)
    ws = torch.empty((nb,), dtype=torch.uint8, device=dev)

    def call():
        rc = lib.dsa_lightning_indexer_fused(0, qd.data_ptr(), kd.data_ptr(), ksd.data_ptr(), wd.data_ptr(), B, S1,
                                             S2, H, D, None, None, None, 0, 0, 3, K, idx.data_ptr(), val.data_ptr(),
                                             ws.data_ptr(), nb, torch.cuda.current_stream(dev).cuda_stream)
        assert rc == 0

    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        call()
    torch.cuda.current_stream(dev).wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for rep in range(3):
        idx.fill_(5)
        val.zero_()
        ws.fill_(rep)  # stale flags, counts and thresholds everywhere in the workspace
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(idx.view(B, S1, 1, K), di) and torch.equal(val.view(B, S1, 1, K), dv)
