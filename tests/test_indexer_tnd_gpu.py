"""GPU parity of the lightning indexer's packed (TND) layouts and of head counts
that are not a multiple of 16.

The reference pads TND rows to BSND on the host
(examples/deepseek_v4/lightning_indexer.py:48-190, 1257-1368); the kernels here
address packed rows in place.  Checks:

* TND logits equal the padded-BSND logits of the same kernel bit for bit
  (row (b, t) of the padded call is packed row cu_q[b-1] + t), and the oracle's
  within the indexer tolerance (1e-2 relative, as in test_indexer_gpu.py);
* TND + PA_BSND keys give the same logits and indices as TND + TND keys;
* the top-k of a TND call is bit-exact given the GPU logits;
* the reference's example 3 (TND+TND, B=8, N1=24, S1=64, S2=3072, K=2048,
  mode 0) and example 4 (TND+PA_BSND, B=2, N1=8, q lengths 1024/2048, key
  lengths 4096/8192, block 128, K=2048, mode 0) shapes pass the reference's
  own 3-step check (lightning_indexer.py:1394-1503).
"""
import numpy as np
import pytest
import torch

from oracle import dsa_oracle as ref

pytestmark = pytest.mark.gpu


def _assert_logits(got, want):
    fin = torch.isfinite(want)
    assert torch.equal(fin, torch.isfinite(got)), "mask mismatch"
    rms = want[fin].double().pow(2).mean().sqrt().item() if fin.any() else 1.0
    d = (got[fin] - want[fin]).abs()
    bound = 1e-2 * (want[fin].abs() + rms)
    assert torch.all(d <= bound), f"max err {d.max().item()} (rms {rms})"


def _packed(q_lens, k_lens, H, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    T, Tk = sum(q_lens), sum(k_lens)
    qf = torch.randn(T, H, D, generator=g)
    kf = torch.randn(Tk, D, generator=g)
    w = torch.randn(T, H, generator=g) / 8
    if dtype == torch.float8_e4m3fn:
        q = qf.to(torch.float8_e4m3fn)
        k, ks = ref.fp8_quantize_per_token(kf)
    else:
        q, k, ks = qf.to(dtype), kf.to(dtype), None
    cu_q = torch.tensor(np.cumsum(q_lens), dtype=torch.int32)
    cu_k = torch.tensor(np.cumsum(k_lens), dtype=torch.int32)
    return q, k, w, ks, cu_q, cu_k


def _paged(k_pad, s_pad, k_lens, bs, seed):
    """Scatter padded keys [B, S2, D] into a shuffled block pool; -1 past each batch's blocks."""
    B, S2, D = k_pad.shape
    nblk = (S2 + bs - 1) // bs
    perm = torch.randperm(B * nblk, generator=torch.Generator().manual_seed(seed)).to(torch.int32)
    table = torch.full((B, nblk + 1), -1, dtype=torch.int32)
    pool = torch.zeros(B * nblk, bs, 1, D, dtype=k_pad.dtype)
    pscale = torch.ones(B * nblk, bs)
    c = 0
    for b in range(B):
        for j in range((k_lens[b] + bs - 1) // bs):
            blk = int(perm[c])
            c += 1
            table[b, j] = blk
            n = min(bs, k_lens[b] - j * bs)
            pool[blk, :n, 0] = k_pad[b, j * bs:j * bs + n]
            if s_pad is not None:
                pscale[blk, :n] = s_pad[b, j * bs:j * bs + n]
    return pool, (pscale if s_pad is not None else None), table


@pytest.mark.parametrize("dtype", [torch.float8_e4m3fn, torch.bfloat16])
@pytest.mark.parametrize("sparse_mode", [3, 0])
def test_tnd_logits_match_padded_and_oracle(dsa, dev, dtype, sparse_mode):
    q_lens, k_lens, H, D = [40, 0, 17, 5], [700, 64, 333, 100], 24, 128
    q, k, w, ks, cu_q, cu_k = _packed(q_lens, k_lens, H, D, dtype, seed=21)
    got = dsa.indexer_logits(q.to(dev), k.unsqueeze(1).to(dev), w.to(dev), None if ks is None else ks.to(dev),
                             actual_seq_lengths_query=cu_q.to(dev), actual_seq_lengths_key=cu_k.to(dev),
                             layout_query="TND", layout_key="TND", sparse_mode=sparse_mode).cpu()
    assert got.shape == (sum(q_lens), max(k_lens))
    # Same kernel on the padded layout: identical rows.
    qp, _ = ref.tnd_to_padded(q.view(torch.uint8), cu_q.tolist())
    kp, _ = ref.tnd_to_padded(k.view(torch.uint8), cu_k.tolist())
    wp, _ = ref.tnd_to_padded(w, cu_q.tolist())
    sp = None if ks is None else ref.tnd_to_padded(ks, cu_k.tolist())[0]
    qp, kp = qp.view(dtype), kp.view(dtype)
    pad = dsa.indexer_logits(qp.to(dev), kp.unsqueeze(2).to(dev), wp.to(dev), None if sp is None else sp.to(dev),
                             actual_seq_lengths_query=torch.tensor(q_lens, dtype=torch.int32).to(dev),
                             actual_seq_lengths_key=torch.tensor(k_lens, dtype=torch.int32).to(dev),
                             sparse_mode=sparse_mode).cpu()
    assert torch.equal(got, ref.padded_to_tnd(pad, q_lens))
    want = ref.lightning_indexer_tnd(q, k, w, cu_q.tolist(), ks, cu_k=cu_k.tolist(), sparse_count=8,
                                     sparse_mode=sparse_mode)[2]
    _assert_logits(got, want)


def test_tnd_topk_and_paged_keys(dsa, dev):
    q_lens, k_lens, H, D, K, bs = [33, 64, 1, 0, 20], [1500, 2600, 70, 9, 2048], 64, 128, 512, 64
    q, k, w, ks, cu_q, cu_k = _packed(q_lens, k_lens, H, D, torch.float8_e4m3fn, seed=22)
    qd, kd, wd, ksd = q.to(dev), k.unsqueeze(1).to(dev), w.to(dev), ks.to(dev)
    cqd, ckd = cu_q.to(dev), cu_k.to(dev)
    kw = dict(actual_seq_lengths_query=cqd, layout_query="TND", sparse_mode=3)
    logits = dsa.indexer_logits(qd, kd, wd, ksd, actual_seq_lengths_key=ckd, layout_key="TND", **kw)
    idx, val = dsa.lightning_indexer(qd, kd, wd, key_scale=ksd, actual_seq_lengths_key=ckd, layout_key="TND",
                                     sparse_count=K, return_value=True, **kw)
    T = sum(q_lens)
    assert idx.shape == (T, 1, K) and val.shape == (T, 1, K)
    ri, rv = ref.topk_stable(logits.cpu(), K)
    assert torch.equal(idx.cpu().view(T, K), ri)
    assert torch.equal(val.cpu().view(T, K), rv)
    # Paged keys with per-batch lengths: the same logits and indices.
    kp, _ = ref.tnd_to_padded(k.view(torch.uint8), cu_k.tolist())
    sp, _ = ref.tnd_to_padded(ks, cu_k.tolist())
    pool, pscale, table = _paged(kp.view(torch.float8_e4m3fn), sp, k_lens, bs, seed=4)
    akd = torch.tensor(k_lens, dtype=torch.int32).to(dev)
    lp = dsa.indexer_logits(qd, pool.to(dev), wd, pscale.to(dev), actual_seq_lengths_key=akd,
                            block_table=table.to(dev), layout_key="PA_BSND", **kw)
    assert torch.equal(lp.cpu(), logits.cpu())
    ip, _ = dsa.lightning_indexer(qd, pool.to(dev), wd, key_scale=pscale.to(dev), actual_seq_lengths_key=akd,
                                  block_table=table.to(dev), layout_key="PA_BSND", sparse_count=K, **kw)
    assert torch.equal(ip.cpu(), idx.cpu())


def test_tnd_validation(dsa, dev):
    q = torch.zeros(10, 16, 128, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(12, 1, 128, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(10, 16, device=dev)
    cu = torch.tensor([4, 10], dtype=torch.int32, device=dev)
    with pytest.raises(ValueError, match="must equal layout_key"):
        dsa.lightning_indexer(q, k, w, actual_seq_lengths_query=cu, actual_seq_lengths_key=cu,
                              layout_query="TND", layout_key="BSND")
    with pytest.raises(ValueError, match="beyond"):
        dsa.lightning_indexer(q, k, w, actual_seq_lengths_query=torch.tensor([4, 11], device=dev),
                              actual_seq_lengths_key=cu, layout_query="TND", layout_key="TND")
    with pytest.raises(ValueError, match="non-decreasing"):
        dsa.lightning_indexer(q, k, w, actual_seq_lengths_query=torch.tensor([6, 4], device=dev),
                              actual_seq_lengths_key=cu, layout_query="TND", layout_key="TND")
    # Empty keys everywhere: the reference's early exit, T rows of -1.
    idx, val = dsa.lightning_indexer(q, k, w, actual_seq_lengths_query=cu,
                                     actual_seq_lengths_key=torch.tensor([0, 0], device=dev),
                                     layout_query="TND", layout_key="TND", sparse_count=16, return_value=True)
    assert idx.shape == (10, 1, 16) and torch.all(idx == -1) and torch.all(torch.isneginf(val))


def _three_step(g_idx, g_scores, tl_idx, thres=1e-4):
    """The reference's step 2 (lightning_indexer.py:1441-1465): every index in
    the symmetric difference of a row's sets has a golden score within `thres`
    relative of the row's K-th golden score."""
    fails = 0
    for r in range(g_idx.shape[0]):
        a = {int(x) for x in g_idx[r].tolist() if x >= 0}
        b = {int(x) for x in tl_idx[r].tolist() if x >= 0}
        if a == b:
            continue
        row = g_scores[r]
        bm = min(row[i].item() for i in a) if a else float("-inf")
        for j in a ^ b:
            sc = row[j].item()
            if bm == 0:
                re = 0.0 if sc == 0 else float("inf")
            elif bm == float("-inf"):
                re = 0.0 if sc <= -1e30 else float("inf")
            else:
                re = abs(sc - bm) / abs(bm)
            fails += re > thres
    return fails


def _uniform(shape, g, dtype=torch.float16):
    return (torch.rand(shape, generator=g, dtype=torch.float64) * 2 - 1).to(dtype)


def test_reference_example_tnd_tnd(dsa, dev):
    B, S1, S2, N1, D, K = 8, 64, 3072, 24, 128, 2048
    g = torch.Generator().manual_seed(42)
    q = _uniform((B * S1, N1, D), g)
    k = _uniform((B * S2, 1, D), g)
    w = _uniform((B * S1, N1), g).abs()
    asq = torch.cumsum(torch.full((B,), S1, dtype=torch.int32), 0)
    ask = torch.cumsum(torch.full((B,), S2, dtype=torch.int32), 0)
    idx, val = dsa.lightning_indexer(q.to(dev), k.to(dev), w.to(dev), actual_seq_lengths_query=asq.to(dev),
                                     actual_seq_lengths_key=ask.to(dev), layout_query="TND", layout_key="TND",
                                     sparse_count=K, sparse_mode=0, return_value=True)
    gi, gv, gl = ref.lightning_indexer_tnd(q, k, w, asq.tolist(), cu_k=ask.tolist(), sparse_count=K, sparse_mode=0)
    assert idx.shape == (B * S1, 1, K) and val.dtype == torch.float16
    assert _three_step(gi.view(-1, K), gl, idx.cpu().view(-1, K)) == 0
    # Step 3: sorted values as fp16, >= 95% within rtol 5e-3 / atol 2.5e-5.
    gs = torch.sort(gv.view(-1, K), dim=1, descending=True)[0].half().float()
    ts = torch.sort(val.cpu().float().view(-1, K), dim=1, descending=True)[0].half().float()
    close = torch.isclose(gs, ts, rtol=5e-3, atol=2.5e-5, equal_nan=True)
    assert close.float().mean().item() >= 0.95


def test_reference_example_tnd_paged(dsa, dev):
    B, N1, D, K, bs = 2, 8, 128, 2048, 128
    act_q, act_k = [1024, 2048], [4096, 8192]
    g = torch.Generator().manual_seed(43)
    q = _uniform((sum(act_q), N1, D), g)
    w = _uniform((sum(act_q), N1), g).abs()
    k_pad = _uniform((B, max(act_k), D), g)
    pool, _, table = _paged(k_pad, None, act_k, bs, seed=42)
    asq = torch.cumsum(torch.tensor(act_q, dtype=torch.int32), 0)
    ask = torch.tensor(act_k, dtype=torch.int32)
    idx, _ = dsa.lightning_indexer(q.to(dev), pool.to(dev), w.to(dev), actual_seq_lengths_query=asq.to(dev),
                                   actual_seq_lengths_key=ask.to(dev), block_table=table.to(dev),
                                   layout_query="TND", layout_key="PA_BSND", sparse_count=K, sparse_mode=0)
    gi, _, gl = ref.lightning_indexer_tnd(q, k_pad, w, asq.tolist(), actual_k_len=act_k, sparse_count=K,
                                          sparse_mode=0)
    assert idx.shape == (sum(act_q), 1, K)
    assert _three_step(gi.view(-1, K), gl, idx.cpu().view(-1, K)) == 0


def test_tnd_fused_topk_equals_dense(dsa, dev):
    """Packed queries with the top-k streamed out of the indexer (dsa_lightning_indexer_tnd_fused):
    bit-equal to the dense TND path, for packed and for paged keys, with an empty batch."""
    q_lens, k_lens, H, D, K, bs = [33, 64, 0, 20], [20000, 40000, 9, 17000], 64, 128, 2048, 64
    print("tnd fused top-k", flush=True)
    q, k, w, ks, cu_q, cu_k = _packed(q_lens, k_lens, H, D, torch.float8_e4m3fn, seed=23)
    qd, kd, wd, ksd = q.to(dev), k.unsqueeze(1).to(dev), w.to(dev), ks.to(dev)
    cqd, ckd = cu_q.to(dev), cu_k.to(dev)
    kw = dict(actual_seq_lengths_query=cqd, layout_query="TND", sparse_mode=3, sparse_count=K)
    di, dv = dsa.lightning_indexer(qd, kd, wd, key_scale=ksd, actual_seq_lengths_key=ckd, layout_key="TND",
                                   return_value=True, fuse_topk=False, **kw)
    fi, fv = dsa.lightning_indexer(qd, kd, wd, key_scale=ksd, actual_seq_lengths_key=ckd, layout_key="TND",
                                   return_value=True, fuse_topk=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(fi, di) and torch.equal(fv, dv)
    kp, _ = ref.tnd_to_padded(k.view(torch.uint8), cu_k.tolist())
    sp, _ = ref.tnd_to_padded(ks, cu_k.tolist())
    pool, pscale, table = _paged(kp.view(torch.float8_e4m3fn), sp, k_lens, bs, seed=5)
    akd = torch.tensor(k_lens, dtype=torch.int32).to(dev)
    pi, _ = dsa.lightning_indexer(qd, pool.to(dev), wd, key_scale=pscale.to(dev), actual_seq_lengths_key=akd,
                                  block_table=table.to(dev), layout_key="PA_BSND", fuse_topk=True, **kw)
    assert torch.equal(pi.cpu(), di.cpu())
