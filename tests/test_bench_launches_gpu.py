"""GPU parity of the C2 and C3 launches themselves, on the very inputs bench.py times.

* C2 (indexer + top-k alone: 4096 query rows x 32768 keys, 64 fp8 heads x 128, per-key scale,
  causal, top-2048): the whole logits launch runs once; 16 rows spread over it (both ends
  included) are compared with the oracle's logits; the dense and the streamed (fused) top-k of
  the launch both equal topk_stable of the GPU logits on every one of the 4096 rows.
* C3 (paged decode: 64 sequences x 65536 keys in 64-token blocks under a random block table,
  128 heads, top-2048): the whole launch runs once through the C ABI with the block table, as
  bench.py calls it; 8 sequences are compared with the oracle on a compact copy of each
  sequence's selected rows, gathered through the table on the host side of the test.

Bars: logits within 1e-2 relative (|d| <= 1e-2 (|ref| + rms(ref))); top-k bit-exact given the
GPU logits; out within atol = rtol = 2e-2, LSE within 1e-3.
"""
import pytest
import torch

import bench
from oracle import dsa_oracle as ref

pytestmark = pytest.mark.gpu

SM = 576 ** -0.5


def _log(msg):
    print(f"[bench-launches] {msg}", flush=True)


def _assert_logits(got, want):
    fin = torch.isfinite(want)
    assert torch.equal(fin, torch.isfinite(got)), "mask mismatch"
    rms = want[fin].double().pow(2).mean().sqrt().item() if fin.any() else 1.0
    d = (got[fin] - want[fin]).abs()
    bound = 1e-2 * (want[fin].abs() + rms)
    assert torch.all(d <= bound), f"max err {d.max().item()} (rms {rms})"


def test_c2_launch_logits_and_topk(dsa, dev):
    q, k, w, ks = bench.gen_indexer(torch, dev)
    S1, S2, K = q.shape[1], k.shape[1], 2048
    _log("C2 logits launch")
    logits = dsa.indexer_logits(q, k, w, ks, sparse_mode=3)
    rows = sorted({int(round(i * (S1 - 1) / 15)) for i in range(16)})
    lg_all = logits[0].cpu()
    lg = lg_all[rows]
    del logits
    _log("C2 oracle logits")
    kc, ksc = k.cpu(), ks.cpu()
    for n, r in enumerate(rows):
        want = ref.indexer_logits(q[:, r:r + 1].cpu(), kc, w[:, r:r + 1].cpu(), ksc, actual_q_len=[1],
                                  actual_k_len=[S2 - S1 + r + 1], sparse_mode=3)[0, 0]
        _assert_logits(lg[n], want)  # keys past the causal bound: -inf in both
    _log("C2 top-k, dense and fused")
    di, dv = dsa.lightning_indexer(q, k, w, key_scale=ks, sparse_count=K, sparse_mode=3, return_value=True,
                                   fuse_topk=False)
    fi, fv = dsa.lightning_indexer(q, k, w, key_scale=ks, sparse_count=K, sparse_mode=3, return_value=True,
                                   fuse_topk=True)
    torch.cuda.synchronize()
    _log("C2 oracle top-k of the GPU logits, every row")
    ri, rv = ref.topk_stable(lg_all, K)
    for name, (i, v) in (("dense", (di, dv)), ("fused", (fi, fv))):
        i, v = i[0, :, 0].cpu(), v[0, :, 0].cpu()
        bad = (i != ri).any(1)
        assert not bad.any(), f"{name}: {int(bad.sum())} rows differ, first {int(bad.nonzero()[0])}"
        assert torch.equal(v, rv), name


def test_c3_decode_launch(dsa, dev):
    from tilelang_ascend_amd import _lib as L

    qd, pool, table, idd, lens = bench.gen_decode(torch, dev)
    B, H, topk = qd.shape[0], qd.shape[2], idd.shape[-1]
    nblk, bs = table.shape[1], pool.shape[1]
    lib = L.load_library()
    out = torch.empty(B, 1, H, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, 1, H, dtype=torch.float32, device=dev)
    ws_bytes = lib.dsa_sparse_mla_workspace_size(B, 1, H, topk)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    _log("C3 launch")
    rc = lib.dsa_sparse_mla_fwd(L.KIND_BF16, qd.data_ptr(), pool.data_ptr(), idd.data_ptr(), table.data_ptr(), None,
                                lens.data_ptr(), B, 1, H, 576, 512, nblk * bs, bs, nblk, topk, SM, 1, out.data_ptr(),
                                lse.data_ptr(), ws.data_ptr(), ws_bytes, L.stream_handle(dev))
    L.check(rc, "decode")
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    seqs = [0, 1, 17, 31, 32, 45, 62, 63]
    _log(f"C3 oracle on sequences {seqs}")
    s = torch.tensor(seqs, device=dev)
    sel = idd.view(B, topk)[s].long()
    phys = table.long()[s].gather(1, torch.div(sel, bs, rounding_mode="floor")) * bs + sel % bs
    rows_kv = pool.view(-1, 576)[phys.view(-1)].view(len(seqs), topk, 1, 576).cpu()
    compact = torch.arange(topk, dtype=torch.int32).view(1, 1, 1, topk).expand(len(seqs), 1, 1, topk).contiguous()
    ro, rl = ref.sparse_mla_fwd(qd[s].cpu(), rows_kv, compact, SM, actual_seq_lengths_kv=[topk] * len(seqs))
    torch.testing.assert_close(out[s].float().cpu(), ro, atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(lse[s].cpu(), rl, atol=1e-3, rtol=1e-3)
