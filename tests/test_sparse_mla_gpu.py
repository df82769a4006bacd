"""GPU parity of the sparse MLA forward against the CPU oracle.

Tolerance of the path's parity bar: out within atol = rtol = 2e-2 (bf16), lse within 1e-3.
"""
import math

import pytest
import torch

from oracle import dsa_oracle as ref

pytestmark = pytest.mark.gpu


def _inputs(B, S, Skv, H, topk, seed, dtype=torch.bfloat16, q_start=None):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, S, H, 576, generator=g) * 0.5).to(dtype)
    kv = (torch.randn(B, Skv, 1, 576, generator=g) * 0.5).to(dtype)
    idx = ref.causal_sparse_indices(B, S, Skv, topk, seed=seed, q_start=q_start)
    return q, kv, idx


def _check(out, lse, ro, rl):
    torch.testing.assert_close(out.float().cpu(), ro, atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(lse.cpu(), rl, atol=1e-3, rtol=1e-3)


def test_config1_parity(dsa, dev):
    # The CPU-runnable case C1: B=1, Sq=128, Skv=4096, H=16, topk=512.
    q, kv, idx = _inputs(1, 128, 4096, 16, 512, seed=20261201)
    out, lse = dsa.sparse_mla_fwd(q.to(dev), kv.to(dev), idx.to(dev), 1 / math.sqrt(576))
    _check(out, lse, *ref.sparse_mla_fwd(q, kv, idx))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_shaped_launch(dsa, dev, dtype):
    # 768 rows x 16 heads: more workgroups than the decode-shaped (single-phase) loop takes, so
    # this runs the two-phase software pipeline that the prefill benchmarks use.
    q, kv, idx = _inputs(1, 768, 4096, 16, 256, seed=21, dtype=dtype)
    out, lse = dsa.sparse_mla_fwd(q.to(dev), kv.to(dev), idx.to(dev), 1 / math.sqrt(576))
    _check(out, lse, *ref.sparse_mla_fwd(q, kv, idx))


@pytest.mark.parametrize("H", [32, 48, 64, 128, 160, 256])
def test_head_counts(dsa, dev, H):
    q, kv, idx = _inputs(1, 4, 2048, H, 256, seed=H)
    out, lse = dsa.sparse_mla_fwd(q.to(dev), kv.to(dev), idx.to(dev))
    _check(out, lse, *ref.sparse_mla_fwd(q, kv, idx))


def test_fp16_inputs(dsa, dev):
    q, kv, idx = _inputs(1, 8, 1024, 128, 256, seed=3, dtype=torch.float16)
    out, lse = dsa.sparse_mla_fwd(q.to(dev), kv.to(dev), idx.to(dev))
    assert out.dtype == torch.float16
    _check(out, lse, *ref.sparse_mla_fwd(q, kv, idx))


def test_decode_paged_h128_topk2048(dsa, dev):
    # Decode shape: B sequences x 1 query, 128 heads, topk 2048 over a paged pool.
    B, Skv, H, topk, bs = 4, 8192, 128, 2048, 64
    g = torch.Generator().manual_seed(31)
    q = (torch.randn(B, 1, H, 576, generator=g) * 0.5).to(torch.bfloat16)
    nblk = Skv // bs
    pool = (torch.randn(B * nblk, bs, 1, 576, generator=g) * 0.5).to(torch.bfloat16)
    table = torch.randperm(B * nblk, generator=g).view(B, nblk).to(torch.int32)
    idx = torch.stack([torch.randperm(Skv, generator=g)[:topk] for _ in range(B)]).view(B, 1, 1, topk).to(torch.int32)
    out, lse = dsa.sparse_mla_fwd(q.to(dev), pool.to(dev), idx.to(dev), block_table=table.to(dev))
    _check(out, lse, *ref.sparse_mla_fwd(q, pool, idx, block_table=table))


def test_padding_causal_and_actual_lengths(dsa, dev):
    B, S, Skv, H, topk = 2, 16, 256, 64, 64
    q, kv, idx = _inputs(B, S, Skv, H, topk, seed=5)
    idx[0, 3, 0, 10:] = -1                  # padded slots
    idx[0, 4, 0, :] = -1                    # empty row -> out 0, lse -inf
    idx[1, 5, 0, :8] = Skv - 1              # future positions masked by causality (duplicates dropped)
    idx[1, 5, 0, 1:8] = -1
    ql = torch.tensor([16, 12], dtype=torch.int32)
    kl = torch.tensor([256, 200], dtype=torch.int32)
    out, lse = dsa.sparse_mla_fwd(q.to(dev), kv.to(dev), idx.to(dev), actual_seq_lengths_query=ql.to(dev),
                                  actual_seq_lengths_kv=kl.to(dev))
    ro, rl = ref.sparse_mla_fwd(q, kv, idx, actual_seq_lengths_query=ql.tolist(), actual_seq_lengths_kv=kl.tolist())
    _check(out, lse, ro, rl)
    assert torch.all(out[0, 4].cpu() == 0) and torch.all(torch.isneginf(lse[0, 4].cpu()))


@pytest.mark.parametrize("topk", [40, 300, 1500])
@pytest.mark.parametrize("paged", [False, True])
def test_decode_rows_edges(dsa, dev, topk, paged):
    # At most 8 query rows: the decode kernel (one workgroup per row and 16 heads up to
    # 256 slots, 128-slot chunks and a combine past that).  Padded rows (out 0, lse -inf),
    # key lengths, the causal bound, -1 and out-of-range slots, an empty 128-slot chunk, fp16.
    B, S, Skv, H, bs = 2, 3, 1800, 32, 48
    for dtype in (torch.bfloat16, torch.float16):
        print(f"sparse_mla decode rows topk={topk} paged={paged} {dtype}", flush=True)
        g = torch.Generator().manual_seed(topk + paged)
        q = (torch.randn(B, S, H, 576, generator=g) * 0.5).to(dtype)
        kv = (torch.randn(B, Skv, 1, 576, generator=g) * 0.5).to(dtype)
        idx = torch.stack([torch.randperm(Skv, generator=g)[:topk] for _ in range(B * S)]).view(B, S, 1, topk)
        idx = idx.to(torch.int32)
        idx[0, 0, 0, : topk // 3] = -1                 # leading empty slots (a whole chunk at topk 1500)
        idx[0, 1, 0, 5] = Skv + 7                      # out of range
        if topk > 256:
            idx[1, 0, 0, 128:256] = -1                 # chunk 1 empty
        ql = torch.tensor([3, 2], dtype=torch.int32)   # row (1, 2) padded
        kl = torch.tensor([Skv, 1000], dtype=torch.int32)
        args = dict(actual_seq_lengths_query=ql.to(dev), actual_seq_lengths_kv=kl.to(dev))
        if paged:
            nblk = (Skv + bs - 1) // bs
            table = torch.randperm(B * nblk, generator=g).view(B, nblk).to(torch.int32)
            pool = torch.zeros(B * nblk, bs, 1, 576, dtype=dtype)
            for b in range(B):
                for j in range(nblk):
                    rows = kv[b, j * bs:(j + 1) * bs]
                    pool[table[b, j], :rows.shape[0]] = rows
            out, lse = dsa.sparse_mla_fwd(q.to(dev), pool.to(dev), idx.to(dev), block_table=table.to(dev), **args)
        else:
            out, lse = dsa.sparse_mla_fwd(q.to(dev), kv.to(dev), idx.to(dev), **args)
        ro, rl = ref.sparse_mla_fwd(q, kv, idx, actual_seq_lengths_query=ql.tolist(),
                                    actual_seq_lengths_kv=kl.tolist())
        _check(out, lse, ro, rl)
        assert torch.all(out[1, 2].cpu() == 0) and torch.all(torch.isneginf(lse[1, 2].cpu()))


def test_split_and_unsplit_agree(dsa, dev):
    # 1 token -> the index list is split across workgroups; 512 tokens -> no split.
    q, kv, idx = _inputs(1, 512, 4096, 128, 512, seed=9)
    qd, kvd, idd = q.to(dev), kv.to(dev), idx.to(dev)
    out_all, lse_all = dsa.sparse_mla_fwd(qd, kvd, idd)
    out_one, lse_one = dsa.sparse_mla_fwd(qd[:, 300:301].contiguous(), kvd, idd[:, 300:301].contiguous(),
                                          actual_seq_lengths_query=torch.tensor([1], device=dev),
                                          actual_seq_lengths_kv=torch.tensor([4096 - 511 + 300], device=dev))
    torch.testing.assert_close(out_one.float(), out_all[:, 300:301].float(), atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(lse_one, lse_all[:, 300:301], atol=1e-4, rtol=1e-4)
    ro, rl = ref.sparse_mla_fwd(q[:, 296:304], kv, idx[:, 296:304], actual_seq_lengths_query=[8],
                                actual_seq_lengths_kv=[4096 - 511 + 303])
    _check(out_all[:, 296:304], lse_all[:, 296:304], ro, rl)


def test_single_index_closed_form(dsa, dev):
    q, kv, _ = _inputs(1, 1, 64, 16, 8, seed=1)
    idx = torch.full((1, 1, 1, 64), -1, dtype=torch.int32)
    idx[0, 0, 0, 37] = 21
    out, lse = dsa.sparse_mla_fwd(q.to(dev), kv.to(dev), idx.to(dev))
    assert torch.equal(out[0, 0].cpu(), kv[0, 21, 0, :512].expand(16, 512))
    want = (q[0, 0].double() @ kv[0, 21, 0].double()) / math.sqrt(576)
    torch.testing.assert_close(lse[0, 0].cpu().double(), want, atol=1e-3, rtol=1e-3)


def test_builder_signature(dsa, dev):
    q, kv, idx = _inputs(1, 32, 2048, 128, 256, seed=8)
    kern = dsa.sparse_attention_fwd(heads=128, dim=512, tail_dim=64, topk=256, kv_stride=1)
    out = kern(q.to(dev), kv.to(dev), idx.to(dev))
    ro, _ = ref.sparse_mla_fwd(q, kv, idx)
    torch.testing.assert_close(out.float().cpu(), ro, atol=2e-2, rtol=2e-2)


def _ramp_inputs(jump_log2, H=128, S=2, topk=256, Skv=1024, seed=12):
    """Scores of later index slots exceed the first tile's by ~jump_log2 (base 2)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.zeros(1, S, H, 576)
    q[..., :64] = 1.0
    q += torch.randn(1, S, H, 576, generator=g) * 0.01
    kv = torch.randn(1, Skv, 1, 576, generator=g) * 0.5
    # t = sm_scale * log2(e) * q.k ~= 64 * c / 24 * 1.4427 for a row with c in its first 64 dims
    c = jump_log2 / (64 / 24 * 1.4426950408889634)
    kv[0, 512:, 0, :64] = c
    idx = torch.empty(1, S, 1, topk, dtype=torch.int32)
    for s in range(S):
        low = torch.randperm(512, generator=g)[:topk // 2]
        high = 512 + torch.randperm(Skv - 512 - S, generator=g)[:topk // 2]
        idx[0, s, 0] = torch.cat([low, high]).to(torch.int32)  # first tiles all low
    return q.to(torch.bfloat16), kv.to(torch.bfloat16), idx


@pytest.mark.parametrize("jump", [40.0, 200.0])  # within the fast path's headroom / beyond it (exact fallback)
@pytest.mark.parametrize("S", [1, 300])          # split index list (+combine) / one workgroup per row
def test_large_score_jumps(dsa, dev, jump, S):
    q, kv, idx = _ramp_inputs(jump, S=S)
    out, lse = dsa.sparse_mla_fwd(q.to(dev), kv.to(dev), idx.to(dev))
    ro, rl = ref.sparse_mla_fwd(q, kv, idx)
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    torch.testing.assert_close(out.float().cpu(), ro, atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(lse.cpu(), rl, atol=1e-3, rtol=1e-3)
