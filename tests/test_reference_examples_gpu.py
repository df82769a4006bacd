"""The reference's own example cases for this path, run through this build's entry points
under the reference's own pass criteria (inputs are drawn here at the same shapes, dtypes and
distributions; the reference's RNG call sequences are not reproduced).

* SFA example (examples/sparse_flash_attention/example_sparse_flash_attn.py:295-326): fp16,
  randn, B=1, S=128, SKV=32768, H=128, topk=2048, q_start = 28672, index lists padded with
  SKV (not -1); assert_close(rtol=atol=1e-2) against the golden.
* Paged SFA example (example_sparse_flash_attn_mask_pa.py:398-456): bf16, randn, S=512,
  SKV=32768, 516 blocks x 128, an all-zero block table, row t drawn from randperm(max(1, t))
  and -1 padded, sparse_mode 3; assert_close(rtol=atol=1e-2) against sfa_golden.
* V4 indexer examples 1 (BSND+BSND, B=2, S1=3, S2=32768, N1=64, mode 3) and 2 (BSND+PA_BSND,
  B=2, S1=1, N1=8, key lengths 1024 / 2048, block 128 x 32, mode 0), both top-2048, fp16
  uniform(-1, 1) inputs and |uniform| weights (examples/deepseek_v4/lightning_indexer.py:1574-1600),
  under the reference's 3-step check (:1394-1503).
* sparse_count 6144 and 8192, the largest the reference accepts (:1238-1239), through
  lightning_indexer and the stand-alone top-k (bit-exact given the GPU logits).
"""
import numpy as np
import pytest
import torch

from oracle import dsa_oracle as ref

pytestmark = pytest.mark.gpu


def _log(msg):
    print(f"[examples] {msg}", flush=True)


def _three_step_idx(g_idx, g_scores, tl_idx, thres=1e-4):
    """Step 2 of the reference's check (lightning_indexer.py:1441-1465): every index in the
    symmetric difference of a row's index sets has a golden score within `thres` relative of
    the row's K-th golden score.  Returns the number of failing indices."""
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


def _three_step_values(g_val, tl_val):
    """Step 3 (:1467-1487): sorted top-K values as fp16, >= 95% within rtol 5e-3 / atol 2.5e-5."""
    K = g_val.shape[-1]
    gs = torch.sort(g_val.float().reshape(-1, K), dim=1, descending=True)[0].half().float()
    ts = torch.sort(tl_val.float().cpu().reshape(-1, K), dim=1, descending=True)[0].half().float()
    close = torch.isclose(gs, ts, rtol=5e-3, atol=2.5e-5, equal_nan=True)
    return close.float().mean().item()


def _uniform(shape, g, dtype=torch.float16):
    return (torch.rand(shape, generator=g, dtype=torch.float64) * 2 - 1).to(dtype)


def test_sfa_example_skv_padding(dsa, dev):
    B, S, SKV, H, DQK, topk, q_start = 1, 128, 32768, 128, 576, 2048, 4096 * 7
    g = torch.Generator().manual_seed(0)
    q = torch.randn((B, S, H, DQK), generator=g).to(torch.float16)
    kv = torch.randn((B, SKV, 1, DQK), generator=g).to(torch.float16)
    idx = torch.full((B, S, 1, topk), SKV, dtype=torch.int32)
    for t in range(S):
        i_i = torch.randperm(max(1, t + q_start), generator=g)[:topk]
        idx[0, t, 0, :len(i_i)] = i_i.to(torch.int32)
    kern = dsa.sparse_attention_fwd(heads=H, dim=512, tail_dim=64, topk=topk, kv_stride=1)
    out = kern(q.to(dev), kv.to(dev), idx.to(dev))
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and out.shape == (B, S, H, 512)
    # The golden casts its fp32 result to the input dtype (example_sparse_flash_attn.py:292).
    ro, _ = ref.sparse_mla_fwd(q, kv, idx)
    torch.testing.assert_close(out.cpu(), ro.to(torch.float16), rtol=1e-2, atol=1e-2)
    # The dense scatter-mask golden on two rows agrees with the gather oracle (SKV slots dropped).
    rows = [0, S - 1]
    for r in rows:
        dense = ref.sparse_mla_dense_ref(q[:, r:r + 1], kv, idx[:, r:r + 1], q_start_index_s=q_start + r)
        torch.testing.assert_close(dense, ro[:, r:r + 1], atol=1e-5, rtol=1e-5)


def test_paged_sfa_example(dsa, dev):
    B, S, SKV, H, DQK, topk, block_num, bs = 1, 512, 32 * 1024, 128, 576, 2048, 516, 128
    g = torch.Generator().manual_seed(1)
    q = torch.randn((B, S, H, DQK), generator=g).to(torch.bfloat16)
    kv = torch.randn((block_num, bs, 1, DQK), generator=g).to(torch.bfloat16)
    idx = torch.full((S, 1, topk), -1, dtype=torch.int32)
    for t in range(S):
        i_i = torch.randperm(max(1, t), generator=g)[:topk]
        idx[t, 0, :len(i_i)] = i_i.to(torch.int32)
    table = torch.zeros((B, SKV // bs), dtype=torch.int32)
    aq = torch.tensor([S] * B, dtype=torch.int32)
    ak = torch.tensor([SKV] * B, dtype=torch.int32)
    # The example's call form: func(q, kv, indices [S, 1, topk], actual_q_len, actual_kv_len, block_table).
    kern = dsa.sparse_attention_fwd(heads=H, dim=512, tail_dim=64, topk=topk, kv_stride=1)
    out = kern(q.to(dev), kv.to(dev), idx.to(dev), aq.to(dev), ak.to(dev), table.to(dev))
    torch.cuda.synchronize()
    ro, _ = ref.sparse_mla_fwd(q, kv, idx.unsqueeze(0), DQK ** -0.5, block_table=table,
                               actual_seq_lengths_query=aq.tolist(), actual_seq_lengths_kv=ak.tolist())
    torch.testing.assert_close(out.cpu(), ro.to(torch.bfloat16), rtol=1e-2, atol=1e-2)


def test_v4_indexer_example1_bsnd_bsnd(dsa, dev):
    B, S1, S2, N1, D, K, mode = 2, 3, 32768, 64, 128, 2048, 3
    g = torch.Generator().manual_seed(42)
    q = _uniform((B, S1, N1, D), g)
    k = _uniform((B, S2, 1, D), g)
    w = _uniform((B, S1, N1), g).abs()
    asq = torch.full((B,), S1, dtype=torch.int32)
    ask = torch.full((B,), S2, dtype=torch.int32)
    idx, val = dsa.lightning_indexer(q.to(dev), k.to(dev), w.to(dev), actual_seq_lengths_query=asq.to(dev),
                                     actual_seq_lengths_key=ask.to(dev), layout_query="BSND", layout_key="BSND",
                                     sparse_count=K, sparse_mode=mode, return_value=True)
    torch.cuda.synchronize()
    gi, gv, gl = ref.lightning_indexer(q, k, w, actual_q_len=asq.tolist(), actual_k_len=ask.tolist(),
                                       sparse_count=K, sparse_mode=mode)
    assert idx.shape == (B, S1, 1, K) and val.dtype == torch.float16
    assert _three_step_idx(gi.view(-1, K), gl.view(-1, S2), idx.cpu().view(-1, K)) == 0
    assert _three_step_values(gv, val) >= 0.95


def _build_pa(k_pad, act_k, bs, block_num, seed=42):
    """Scatter padded keys [B, S2, 1, D] into a pool [block_num, bs, 1, D] through a table
    [B, block_num] of a random block permutation, -1 past each batch's blocks (the reference's
    _build_pa, lightning_indexer.py:1505-1530)."""
    B, S2, _, D = k_pad.shape
    perm = np.random.RandomState(seed).permutation(block_num).astype(np.int32)
    table = torch.full((B, block_num), -1, dtype=torch.int32)
    pool = torch.zeros((block_num, bs, 1, D), dtype=k_pad.dtype)
    c = 0
    for b in range(B):
        for i in range((act_k[b] + bs - 1) // bs):
            blk = int(perm[c])
            c += 1
            table[b, i] = blk
            n = min(bs, act_k[b] - i * bs)
            pool[blk, :n] = k_pad[b, i * bs:i * bs + n]
    return pool, table


def test_v4_indexer_example2_bsnd_paged(dsa, dev):
    B, S1, N1, D, K, mode, bs, block_num = 2, 1, 8, 128, 2048, 0, 128, 32
    act_k = [1024, 2048]
    g = torch.Generator().manual_seed(43)
    q = _uniform((B, S1, N1, D), g)
    w = _uniform((B, S1, N1), g).abs()
    k_pad = _uniform((B, max(act_k), 1, D), g)
    pool, table = _build_pa(k_pad, act_k, bs, block_num)
    asq = torch.full((B,), S1, dtype=torch.int32)
    ask = torch.tensor(act_k, dtype=torch.int32)
    idx, _ = dsa.lightning_indexer(q.to(dev), pool.to(dev), w.to(dev), actual_seq_lengths_query=asq.to(dev),
                                   actual_seq_lengths_key=ask.to(dev), block_table=table.to(dev),
                                   layout_query="BSND", layout_key="PA_BSND", sparse_count=K, sparse_mode=mode)
    torch.cuda.synchronize()
    gi, _, gl = ref.lightning_indexer(q, k_pad, w, actual_q_len=asq.tolist(), actual_k_len=act_k,
                                      sparse_count=K, sparse_mode=mode)
    got = idx.cpu().view(-1, K)
    assert _three_step_idx(gi.view(-1, K), gl.view(-1, max(act_k)), got) == 0
    # Batch 0 has 1024 keys: its list ends in 1024 slots of -1.
    assert torch.all(got[0, 1024:] == -1) and torch.all(got[0, :1024] >= 0) and torch.all(got[1] >= 0)


def _boundary_fails(g_idx, g_scores, tl_idx, rel=1e-2):
    """Step 2 with the fp8 indexer's logits bar in place of 1e-4: every index in the symmetric
    difference of a row's sets has a golden score within rel * (|K-th score| + rms(row)) of the
    row's K-th golden score (fp8 logits are only pinned to 1e-2 relative)."""
    fails = 0
    for r in range(g_idx.shape[0]):
        a = {int(x) for x in g_idx[r].tolist() if x >= 0}
        b = {int(x) for x in tl_idx[r].tolist() if x >= 0}
        if a == b:
            continue
        row = g_scores[r]
        fin = torch.isfinite(row)
        rms = row[fin].double().pow(2).mean().sqrt().item()
        bm = min(row[i].item() for i in a)
        fails += sum(abs(row[j].item() - bm) > rel * (abs(bm) + rms) for j in a ^ b)
    return fails


@pytest.mark.parametrize("dtype", [torch.float16, torch.float8_e4m3fn])
@pytest.mark.parametrize("K", [6144, 8192])
def test_indexer_sparse_count_beyond_4096(dsa, dev, K, dtype):
    """lightning_indexer at the largest sparse counts the reference accepts: batch 0 has fewer
    valid keys than K (-1 padding), batch 1 more; indices and values bit-exact against the
    stable top-k of the GPU logits, and against the oracle's logits the reference's step 2
    (fp16, the reference's own inputs: 1e-4 of the K-th score) or the fp8 logits bar (1e-2)."""
    B, S1, S2, H, D = 2, 24, 20000, 64, 128
    g = torch.Generator().manual_seed(K)
    if dtype == torch.float16:
        q = _uniform((B, S1, H, D), g)
        k = _uniform((B, S2, D), g)
        w = _uniform((B, S1, H), g).abs()
        ks = None
    else:
        q = torch.randn(B, S1, H, D, generator=g).to(torch.float8_e4m3fn)
        k, ks = ref.fp8_quantize_per_token(torch.randn(B, S2, D, generator=g))
        w = torch.randn(B, S1, H, generator=g) / 8
    ak = torch.tensor([5000, S2], dtype=torch.int32)
    qd, kd, wd, akd = q.to(dev), k.unsqueeze(2).to(dev), w.to(dev), ak.to(dev)
    ksd = None if ks is None else ks.to(dev)
    kw = dict(actual_seq_lengths_key=akd, sparse_mode=3)
    logits = dsa.indexer_logits(qd, kd, wd, ksd, **kw)
    idx, val = dsa.lightning_indexer(qd, kd, wd, key_scale=ksd, sparse_count=K, return_value=True, **kw)
    torch.cuda.synchronize()
    ri, rv = ref.topk_stable(logits.cpu().view(B * S1, S2), K)
    assert torch.equal(idx.cpu().view(B * S1, K), ri)
    assert torch.equal(val.cpu().float().view(B * S1, K), rv.to(val.dtype).float())
    got = idx.cpu().view(B, S1, K)
    assert torch.all(got[0, :, 5000:] == -1)
    gi, _, gl = ref.lightning_indexer(q, k, w, ks, actual_k_len=ak.tolist(), sparse_count=K, sparse_mode=3)
    if dtype == torch.float16:
        assert _three_step_idx(gi.view(-1, K), gl.view(-1, S2), got.view(-1, K)) == 0
    else:
        assert _boundary_fails(gi.view(-1, K), gl.view(-1, S2), got.view(-1, K)) == 0


@pytest.mark.parametrize("n", [16384, 100000])
@pytest.mark.parametrize("K", [6144, 8192])
def test_topk_selector_k_beyond_4096(dsa, dev, n, K):
    g = torch.Generator().manual_seed(n + K)
    x = torch.randn(12, n, generator=g)
    x[1] = torch.round(x[1] * 4) / 4                      # heavy ties: lower index wins
    x[2, 3000:] = float("-inf")                            # fewer than K finite scores
    x[3] = 0.0                                             # one constant row
    x[4, ::7] = float("nan")                               # NaN never takes a slot
    xd = x.to(dev)
    idx, val = dsa.topk_selector(xd, K, sorted=True, return_values=True)
    torch.cuda.synchronize()
    ri, rv = ref.topk_stable(x, K)
    assert torch.equal(idx.cpu(), ri)
    assert torch.equal(val.cpu(), rv)
