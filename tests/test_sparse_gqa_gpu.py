"""GPU parity of sparse attention over KV groups against the grouped oracle.

* The 128-wide grouped kernel (examples/sparse_flash_attention/example_sparse_flash_attn_gqa.py:13-295,
  K = V = the whole row): the example's own inputs and check, random inputs at its shape,
  head counts per group from 8 to 64, causal rows, -1 padding, query / key lengths, ragged
  and maximal topk.
* kv_group > 1 through the 576-wide kernels (example_sparse_flash_attn.py:19-46 with kv
  [B, Skv, kv_group, 576]): prefill-shaped rows (the gather kernel), decode rows (the decode
  kernel), a paged pool, and the builder.

Tolerances: out within atol = rtol = 1e-2 (fp16; the example's own bar) or 2e-2 (bf16); lse
within 1e-3.
"""
import pytest
import torch

from oracle import dsa_oracle as ref

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def _grouped_indices(B, S, G, Skv, topk, seed, pad_frac=0.25, bad_frac=0.05, q_start=None):
    """[B, S, G, topk] int32: per (row, group) distinct positions, most within the causal bound
    (q_start + t, default Skv - S + t), some beyond it or past Skv, a tail of -1."""
    g = torch.Generator().manual_seed(seed)
    q_start = Skv - S if q_start is None else q_start
    idx = torch.full((B, S, G, topk), -1, dtype=torch.int32)
    for b in range(B):
        for t in range(S):
            lim = q_start + t + 1
            for k in range(G):
                n = min(topk, lim)
                n = max(1, int(n * (1 - pad_frac * float(torch.rand(1, generator=g)))))
                sel = torch.randperm(lim, generator=g)[:n]
                nbad = int(n * bad_frac)
                if nbad and lim < Skv:
                    sel[:nbad] = torch.randint(lim, Skv + 3, (nbad,), generator=g).to(sel.dtype)
                    sel = torch.unique(sel)[:n]
                    sel = sel[torch.randperm(sel.numel(), generator=g)]
                idx[b, t, k, :sel.numel()] = sel.to(torch.int32)
    return idx


def _check(out, lse, ro, rl, dtype):
    tol = 1e-2 if dtype == torch.float16 else 2e-2
    torch.testing.assert_close(out.float().cpu(), ro, atol=tol, rtol=tol)
    lse = lse.cpu()
    fin = torch.isfinite(rl)
    assert torch.equal(torch.isfinite(lse), fin)
    torch.testing.assert_close(lse[fin], rl[fin], atol=1e-3, rtol=1e-3)


def test_gqa_reference_example(dsa, dev):
    """The example's own inputs (B=2, S=273, SKV=44444, 64 query heads over 4 KV heads, D=128,
    topk 2048, fp16, q_start 28672; every KV row of a head equal, :276-318) and its check
    (rtol = atol = 1e-2 against the golden, whose output is then that head's row), then the
    same shape with random KV rows against the oracle."""
    B, S, SKV, HQ, HKV, D, topk = 2, 273, 44444, 64, 4, 128, 2048
    q_start = 4096 * 7
    g = torch.Generator().manual_seed(0)
    q = torch.randn(B, S, HQ, D, generator=g).to(torch.float16)
    kv = torch.zeros(B, SKV, HKV, D, dtype=torch.float16)
    for h in range(HKV):
        kv[:, :, h, :] = torch.rand(D, generator=g).to(torch.float16)
    idx = torch.full((B, S, HKV, topk), SKV, dtype=torch.int32)
    for b in range(B):
        for t in range(S):
            for h in range(HKV):
                i_i = torch.randperm(max(1, t + q_start), generator=g)[:topk]
                idx[b, t, h, :len(i_i)] = i_i.to(torch.int32)
    _log("GQA example inputs: constant rows per KV head")
    kern = dsa.sparse_attention_fwd(heads=HQ, dim=D, tail_dim=0, topk=topk, kv_stride=1, kv_group=HKV)
    out = kern(q.to(dev), kv.to(dev), idx.to(dev)).cpu()
    want = kv[0, 0].float().repeat_interleave(HQ // HKV, dim=0).expand(B, S, HQ, D)
    torch.testing.assert_close(out.float(), want, rtol=1e-2, atol=1e-2)

    _log("GQA example shape: random rows against the oracle")
    kv = torch.randn(B, SKV, HKV, D, generator=g).to(torch.float16)
    out, lse = dsa.sparse_gqa_fwd(q.to(dev), kv.to(dev), idx.to(dev))
    ro, rl = ref.sparse_attention_grouped(q, kv, idx, d_v=D)
    _check(out, lse, ro, rl, torch.float16)
    # The example's golden itself (dense scatter mask, causal q_start + t >= j) on a few rows:
    # one row at a time, each with its own causal origin.
    for t in (0, 100, 272):
        dense = ref.sparse_gqa_dense_ref(q[:1, t:t + 1], kv[:1], idx[:1, t:t + 1], q_start_index_s=q_start + t)
        torch.testing.assert_close(out[:1, t:t + 1].float().cpu(), dense, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("G,Hg", [(1, 16), (2, 8), (4, 16), (2, 32), (1, 48), (2, 64)])
def test_gqa_parity(dsa, dev, dtype, G, Hg):
    B, S, Skv, topk = 2, 24, 3000, 512
    g = torch.Generator().manual_seed(1000 * G + Hg)
    q = torch.randn(B, S, G * Hg, 128, generator=g).to(dtype)
    kv = torch.randn(B, Skv, G, 128, generator=g).to(dtype)
    idx = _grouped_indices(B, S, G, Skv, topk, seed=G + Hg)
    _log(f"GQA parity G={G} Hg={Hg} {dtype}")
    out, lse = dsa.sparse_gqa_fwd(q.to(dev), kv.to(dev), idx.to(dev))
    ro, rl = ref.sparse_attention_grouped(q, kv, idx, d_v=128)
    _check(out, lse, ro, rl, dtype)


def test_gqa_lengths_short_rows_and_scale(dsa, dev):
    """Query / key lengths (rows past the query length: out 0, lse -inf), causal rows with
    fewer valid slots than one tile, and an explicit sm_scale."""
    B, S, Skv, G, Hg, topk = 3, 40, 600, 2, 16, 256
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, S, G * Hg, 128, generator=g).to(torch.bfloat16)
    kv = torch.randn(B, Skv, G, 128, generator=g).to(torch.bfloat16)
    idx = _grouped_indices(B, S, G, Skv, topk, seed=6, q_start=2)  # early rows see 3.. keys
    ql, kl = [40, 17, 1], [600, 100, 9]
    _log("GQA lengths")
    out, lse = dsa.sparse_gqa_fwd(q.to(dev), kv.to(dev), idx.to(dev), 0.05,
                                  actual_seq_lengths_query=torch.tensor(ql, dtype=torch.int32),
                                  actual_seq_lengths_kv=torch.tensor(kl, dtype=torch.int32))
    ro, rl = ref.sparse_attention_grouped(q, kv, idx, 0.05, d_v=128, actual_seq_lengths_query=ql,
                                          actual_seq_lengths_kv=kl)
    _check(out, lse, ro, rl, torch.bfloat16)
    assert torch.all(out[1, 17:].float().cpu() == 0) and torch.all(torch.isinf(lse[1, 17:].cpu()))


@pytest.mark.parametrize("topk", [1, 100, 8192])
def test_gqa_ragged_and_max_topk(dsa, dev, topk):
    B, S, Skv, G, Hg = 1, 6, 9000, 2, 16
    g = torch.Generator().manual_seed(topk)
    q = torch.randn(B, S, G * Hg, 128, generator=g).to(torch.float16)
    kv = torch.randn(B, Skv, G, 128, generator=g).to(torch.float16)
    idx = _grouped_indices(B, S, G, Skv, topk, seed=topk, pad_frac=0.1)
    _log(f"GQA topk={topk}")
    out, lse = dsa.sparse_gqa_fwd(q.to(dev), kv.to(dev), idx.to(dev))
    ro, rl = ref.sparse_attention_grouped(q, kv, idx, d_v=128)
    _check(out, lse, ro, rl, torch.float16)


def _mla_group_inputs(B, S, Skv, G, Hg, topk, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, S, G * Hg, 576, generator=g) * 0.5).to(dtype)
    kv = (torch.randn(B, Skv, G, 576, generator=g) * 0.5).to(dtype)
    idx = _grouped_indices(B, S, G, Skv, topk, seed=seed + 1)
    return q, kv, idx


@pytest.mark.parametrize("B,S", [(1, 96), (4, 1)])
def test_mla_kv_groups(dsa, dev, B, S):
    """kv_group 2 with 64 heads per group: 192 query rows of groups (the gather kernel) and
    four decode rows x 2 groups (the decode kernel)."""
    q, kv, idx = _mla_group_inputs(B, S, 2048, 2, 64, 256, seed=31 + B)
    _log(f"MLA kv_group=2 B={B} S={S}")
    out, lse = dsa.sparse_mla_fwd(q.to(dev), kv.to(dev), idx.to(dev))
    ro, rl = ref.sparse_attention_grouped(q, kv, idx, d_v=512)
    _check(out, lse, ro, rl, torch.bfloat16)


def test_mla_kv_groups_paged_and_builder(dsa, dev):
    """A paged pool [blocks, 64, kv_group, 576] through a permuted block table, and the builder's
    kv_group argument on a contiguous cache."""
    B, S, Skv, G, Hg, topk, bs = 2, 12, 1024, 2, 16, 128, 64
    q, kv, idx = _mla_group_inputs(B, S, Skv, G, Hg, topk, seed=77)
    nblk = Skv // bs
    perm = torch.randperm(B * nblk, generator=torch.Generator().manual_seed(78))
    pool = torch.empty(B * nblk, bs, G, 576, dtype=kv.dtype)
    table = torch.empty(B, nblk, dtype=torch.int32)
    for b in range(B):
        for e in range(nblk):
            p = int(perm[b * nblk + e])
            pool[p] = kv[b, e * bs:(e + 1) * bs]
            table[b, e] = p
    ro, rl = ref.sparse_attention_grouped(q, kv, idx, d_v=512)
    _log("MLA kv_group=2 paged")
    out, lse = dsa.sparse_mla_fwd(q.to(dev), pool.to(dev), idx.to(dev), block_table=table.to(dev))
    _check(out, lse, ro, rl, torch.bfloat16)
    _log("MLA kv_group=2 builder")
    kern = dsa.sparse_attention_fwd(heads=G * Hg, dim=512, tail_dim=64, topk=topk, kv_stride=1, kv_group=G)
    out = kern(q.to(dev), kv.to(dev), idx.to(dev))
    torch.testing.assert_close(out.float().cpu(), ro, atol=2e-2, rtol=2e-2)


def test_mla_kv_groups_split_combine(dsa, dev):
    """kv_group 2 on 8 decode rows: 16 (row, group) pairs of 64 heads over topk 2048 take the gather
    kernel with split index lists and the combine (a workspace is needed), against the oracle."""
    B, S, Skv, G, Hg, topk = 8, 1, 8192, 2, 64, 2048
    lib = dsa.load_library()
    assert lib.dsa_sparse_attention_workspace_size(B, S, G * Hg, G, 576, topk) > 0
    q, kv, idx = _mla_group_inputs(B, S, Skv, G, Hg, topk, seed=91)
    _log("MLA kv_group=2 split + combine")
    out, lse = dsa.sparse_mla_fwd(q.to(dev), kv.to(dev), idx.to(dev))
    ro, rl = ref.sparse_attention_grouped(q, kv, idx, d_v=512)
    _check(out, lse, ro, rl, torch.bfloat16)
