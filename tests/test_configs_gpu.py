"""GPU parity at the benchmark configurations' full shapes, on the very inputs bench.py times.

* C4 sparse MLA prefill (B=1, Sq=Skv=16384, H=128, topk=2048, rows i < 2047 padded with -1):
  the whole launch runs once; rows 0-63 and 2040-2055 (-1 padding and where it stops), 64
  seeded random rows and the last 64 rows are compared with the CPU oracle (fp64); every row
  of the launch is checked for the size-independent property that permuting a row's index
  slots leaves its output unchanged (within the bf16 bar), which moves the -1 slots and the
  first valid tile around.
* C5 (128K context): the 4096 x 131072 fp8 indexer (2 GiB of logits, row byte offsets up to
  2^31) on 16 rows spread over the whole buffer against the oracle's logits; the dense
  (two-stage) and the streamed (fused) top-k against topk_stable on the GPU logits, bit for
  bit; sparse MLA on that selection against the oracle on the same rows; and the decode step
  of 32 sequences x 131072 paged keys through indexer -> top-k -> sparse MLA on all 32 rows.

Bars: indexer logits within 1e-2 relative (|d| <= 1e-2 (|ref| + rms(ref))); top-k indices
and values bit-exact given the GPU logits; sparse MLA out within atol = rtol = 2e-2, LSE
within 1e-3.
"""
import pytest
import torch

import bench
from oracle import dsa_oracle as ref

pytestmark = pytest.mark.gpu

SM = 576 ** -0.5


def _log(msg):
    print(f"[configs] {msg}", flush=True)


def _assert_logits(got, want):
    fin = torch.isfinite(want)
    assert torch.equal(fin, torch.isfinite(got)), "mask mismatch"
    rms = want[fin].double().pow(2).mean().sqrt().item() if fin.any() else 1.0
    d = (got[fin] - want[fin]).abs()
    bound = 1e-2 * (want[fin].abs() + rms)
    assert torch.all(d <= bound), f"max err {d.max().item()} (rms {rms})"


def _check_mla(out, lse, ro, rl):
    torch.testing.assert_close(out.float().cpu(), ro, atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(lse.float().cpu(), rl, atol=1e-3, rtol=1e-3)


def _oracle_rows(q, kv_cpu, idx, rows, pos_of_row):
    """Oracle out / lse for query rows `rows` of a B=1 launch whose row r sits at causal position
    pos_of_row(r) (it may see keys 0 .. pos); contiguous runs go in one call."""
    outs, lses = [], []
    i = 0
    while i < len(rows):
        j = i
        while j + 1 < len(rows) and rows[j + 1] == rows[j] + 1:
            j += 1
        r0, r1 = rows[i], rows[j] + 1
        qs = q[:, r0:r1].cpu()
        ids = idx[:, r0:r1].cpu()
        kl = pos_of_row(r1 - 1) + 1
        o, l = ref.sparse_mla_fwd(qs, kv_cpu, ids, SM, actual_seq_lengths_query=[r1 - r0],
                                  actual_seq_lengths_kv=[kl])
        outs.append(o)
        lses.append(l)
        i = j + 1
    return torch.cat(outs, dim=1), torch.cat(lses, dim=1)


# ---------------------------------------------------------------------------------------- C4
@pytest.fixture(scope="module")
def c4(dev):
    _log("C4 inputs")
    q, kv, idx = bench.gen_prefill(torch, dev, S=16384, H=128, topk=2048)
    return q, kv, idx


def test_c4_prefill_launch_sampled_rows(dsa, dev, c4):
    q, kv, idx = c4
    S = q.shape[1]
    _log("C4 launch")
    out, lse = dsa.sparse_mla_fwd(q, kv, idx, SM)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    # Rows 0..2046 hold min(i + 1, 2048) indices: the rest of the list is -1.
    n_valid = (idx[0, :, 0] >= 0).sum(dim=1)
    want_valid = torch.clamp(torch.arange(S, device=dev) + 1, max=2048)
    assert torch.equal(n_valid, want_valid)
    g = torch.Generator().manual_seed(4)
    rand = (torch.randperm(S - 256, generator=g)[:64] + 128).tolist()
    rows = sorted(set(range(0, 64)) | set(range(2040, 2056)) | set(rand) | set(range(S - 64, S)))
    _log(f"C4 oracle on {len(rows)} rows")
    ro, rl = _oracle_rows(q, kv.cpu(), idx, rows, lambda r: r)
    sel = torch.tensor(rows, device=dev)
    _check_mla(out[:, sel], lse[:, sel], ro, rl)


def test_c4_prefill_slot_permutation_invariance(dsa, dev, c4):
    """Every row of the full launch: a random permutation of each row's index slots (the -1 slots
    included) gives the same output within the parity bar."""
    q, kv, idx = c4
    S = q.shape[1]
    out, lse = dsa.sparse_mla_fwd(q, kv, idx, SM)
    g = torch.Generator(device=dev).manual_seed(11)
    perm = torch.argsort(torch.rand(S, idx.shape[-1], generator=g, device=dev), dim=1)
    idx_p = torch.gather(idx[0, :, 0], 1, perm).view_as(idx).contiguous()
    out_p, lse_p = dsa.sparse_mla_fwd(q, kv, idx_p, SM)
    torch.cuda.synchronize()
    _log("C4 permuted launch done")
    d = (out_p.float() - out.float()).abs()
    assert torch.all(d <= 2e-2 + 2e-2 * out.float().abs()), f"max |d| {d.max().item()}"
    dl = (lse_p - lse).abs()
    assert torch.all(dl <= 1e-3 + 1e-3 * lse.abs()), f"max lse |d| {dl.max().item()}"


# ---------------------------------------------------------------------------------------- C5
CTX, CHUNK, TOPK = 131072, 4096, 2048


@pytest.fixture(scope="module")
def c5(dev):
    _log("C5 inputs")
    g = torch.Generator(device=dev).manual_seed(bench.C5_SEED)
    pre = bench.gen_c5_prefill(torch, dev, g, ctx=CTX, chunk=CHUNK)
    dec = bench.gen_c5_decode(torch, dev, g, ctx=CTX, dec_b=32)
    return pre, dec


def _c5_rows():
    # 16 rows spread over the 2 GiB logits buffer (row r starts at byte r * 2^19), both ends included.
    return sorted({int(round(i * (CHUNK - 1) / 15)) for i in range(16)})


def test_c5_indexer_topk_mla_chain(dsa, dev, c5):
    (qi, ki, ks, wi, q, kv), _ = c5
    rows = _c5_rows()
    sel = torch.tensor(rows, device=dev)
    key = ki.view(1, CTX, 1, 128)
    _log("C5 indexer logits")
    logits = dsa.indexer_logits(qi, key, wi, ks, sparse_mode=3)
    lg_rows = logits[0, sel].cpu()
    del logits
    _log("C5 oracle logits")
    k_cpu, ks_cpu = ki.cpu(), ks.cpu()
    for n, r in enumerate(rows):
        pos = CTX - CHUNK + r
        want = ref.indexer_logits(qi[:, r:r + 1].cpu(), k_cpu, wi[:, r:r + 1].cpu(), ks_cpu,
                                  actual_q_len=[1], actual_k_len=[pos + 1], sparse_mode=3)[0, 0]
        _assert_logits(lg_rows[n], want)
    _log("C5 top-k, dense and fused")
    di, dv = dsa.lightning_indexer(qi, key, wi, key_scale=ks, sparse_count=TOPK, sparse_mode=3,
                                   return_value=True, fuse_topk=False)
    fi, fv = dsa.lightning_indexer(qi, key, wi, key_scale=ks, sparse_count=TOPK, sparse_mode=3,
                                   return_value=True, fuse_topk=True)
    torch.cuda.synchronize()
    ri, rv = ref.topk_stable(lg_rows, TOPK)
    assert torch.equal(di[0, sel, 0].cpu(), ri) and torch.equal(dv[0, sel, 0].cpu(), rv)
    assert torch.equal(fi, di) and torch.equal(fv, dv)
    _log("C5 sparse MLA on the selection")
    out, lse = dsa.sparse_mla_fwd(q, kv, fi, SM)
    torch.cuda.synchronize()
    ro, rl = _oracle_rows(q, kv.cpu(), fi, rows, lambda r: CTX - CHUNK + r)
    _check_mla(out[:, sel], lse[:, sel], ro, rl)


def test_c5_decode_chain_all_rows(dsa, dev, c5):
    _, (qd, kd, kds, wd, table, lens_q, lens_k, qm, pool) = c5
    B, bs = qd.shape[0], kd.shape[1]
    _log("C5 decode indexer")
    dlog = dsa.indexer_logits(qd, kd.unsqueeze(2), wd, kds, actual_seq_lengths_query=lens_q,
                              actual_seq_lengths_key=lens_k, block_table=table, layout_key="PA_BSND",
                              sparse_mode=3)
    didx, _ = dsa.lightning_indexer(qd, kd.unsqueeze(2), wd, key_scale=kds, actual_seq_lengths_query=lens_q,
                                    actual_seq_lengths_key=lens_k, block_table=table, layout_key="PA_BSND",
                                    sparse_count=TOPK, sparse_mode=3)
    out, lse = dsa.sparse_mla_fwd(qm, pool, didx, SM, block_table=table, actual_seq_lengths_query=lens_q,
                                  actual_seq_lengths_kv=lens_k)
    torch.cuda.synchronize()
    dlog_c = dlog.view(B, CTX).cpu()
    # Top-k bit-exact given the GPU logits.
    ri, _ = ref.topk_stable(dlog_c, TOPK)
    assert torch.equal(didx.view(B, TOPK).cpu(), ri)
    _log("C5 decode oracle logits")
    tl = table.long()
    kd8 = kd.view(torch.uint8)
    for b in range(B):
        # This sequence's keys in logical order (gathered as bytes: fp8 has no index kernels).
        kb = kd8[tl[b]].reshape(1, CTX, 128).cpu().view(torch.float8_e4m3fn)
        sb = kds[tl[b]].reshape(1, CTX).cpu()
        want = ref.indexer_logits(qd[b:b + 1].cpu(), kb, wd[b:b + 1].cpu(), sb, sparse_mode=3)[0, 0]
        _assert_logits(dlog_c[b], want)
    _log("C5 decode MLA oracle")
    # The oracle on a compact per-sequence copy of the selected rows (slot j -> row j).
    sel = didx.view(B, TOPK).long()
    assert torch.all(sel >= 0)
    phys = tl.gather(1, torch.div(sel, bs, rounding_mode="floor")) * bs + sel % bs
    rows_kv = pool.view(-1, 576)[phys.view(-1)].view(B, TOPK, 1, 576).cpu()
    compact = torch.arange(TOPK, dtype=torch.int32).view(1, 1, 1, TOPK).expand(B, 1, 1, TOPK).contiguous()
    ro, rl = ref.sparse_mla_fwd(qm.cpu(), rows_kv, compact, SM, actual_seq_lengths_kv=[TOPK] * B)
    _check_mla(out, lse, ro, rl)
