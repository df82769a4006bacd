"""Pins the CPU oracle (oracle/dsa_oracle.py) against the reference's known-answer
tests, brute force and closed forms.  CPU only."""
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as ref

GOLDEN = Path(__file__).resolve().parent / "golden"


# --------------------------------------------------------------------------- top-k
def test_topk_kat_sort_arange131():
    d = np.load(GOLDEN / "kat_sort_arange131.npz")
    idx, val = ref.topk_stable(torch.from_numpy(d["x"]), d["x"].shape[1])
    assert np.array_equal(idx.numpy(), d["idx"])
    assert np.array_equal(val.numpy(), d["val"])


def test_topk_kat_topk_arange51():
    d = np.load(GOLDEN / "kat_topk_arange51_k10.npz")
    idx, val = ref.topk_stable(torch.from_numpy(d["x"]), int(d["k"]))
    assert np.array_equal(idx.numpy(), d["idx"])
    assert np.array_equal(val.numpy(), d["val"])


def test_topk_ties_brute_force():
    d = np.load(GOLDEN / "ties_topk.npz")
    idx, val = ref.topk_stable(torch.from_numpy(d["x"]), int(d["k"]))
    assert np.array_equal(idx.numpy(), d["idx"])
    assert np.array_equal(val.numpy(), d["val"])


def test_topk_matches_torch_topk_without_ties():
    g = torch.Generator().manual_seed(0)
    x = torch.stack([torch.randperm(4096, generator=g) for _ in range(64)]).float() * 0.37 - 700.0
    assert all(torch.unique(r).numel() == r.numel() for r in x)
    idx, val = ref.topk_stable(x, 2048)
    tv, ti = torch.topk(x, 2048, dim=1, largest=True, sorted=True)
    assert torch.equal(idx, ti.to(torch.int32))
    assert torch.equal(val, tv)


def test_topk_constant_rows_take_lowest_indices():
    x = torch.full((3, 100), 1.5)
    idx, _ = ref.topk_stable(x, 10)
    assert torch.equal(idx, torch.arange(10, dtype=torch.int32).expand(3, 10))


def test_topk_valid_len_and_padding():
    x = torch.arange(20, dtype=torch.float32).view(1, 20)
    idx, _ = ref.topk_stable(x, 8, valid_len=[5])
    assert idx.tolist() == [[4, 3, 2, 1, 0, -1, -1, -1]]


# --------------------------------------------------------------------------- fp8 quantiser
def test_fp8_quantiser_absmax_and_roundtrip():
    x = torch.tensor([[1.0, -2.0, 0.5, 4.0], [0.0, 0.0, 0.0, 0.0]])
    q, s = ref.fp8_quantize_per_token(x)
    assert s[0].item() == pytest.approx(4.0 / 448.0)
    assert q[0, 3].float().item() == 448.0
    # Values that are exact multiples of the scale by e4m3-representable numbers round-trip.
    assert torch.equal((q[0].float() * s[0]), x[0])
    assert torch.equal(q[1].float(), torch.zeros(4)) and s[1].item() == 1.0


# --------------------------------------------------------------------------- indexer logits
def _brute_logits(q, k, w, scale, sparse_mode):
    B, S1, H, D = q.shape
    S2 = k.shape[1]
    out = torch.full((B, S1, S2), float("-inf"))
    for b in range(B):
        for t in range(S1):
            lim = ref.causal_valid_len(S1, S2, t, sparse_mode)
            for s in range(lim):
                acc = 0.0
                for h in range(H):
                    dot = sum(float(q[b, t, h, d]) * float(k[b, s, d]) for d in range(D))
                    acc += float(w[b, t, h]) * max(dot, 0.0)
                out[b, t, s] = acc * (1.0 if scale is None else float(scale[b, s]))
    return out


@pytest.mark.parametrize("sparse_mode", [0, 3])
def test_indexer_logits_brute_force(sparse_mode):
    g = torch.Generator().manual_seed(1)
    B, S1, S2, H, D = 2, 3, 7, 4, 5
    q = torch.randn(B, S1, H, D, generator=g)
    k = torch.randn(B, S2, D, generator=g)
    w = torch.randn(B, S1, H, generator=g)
    sc = torch.rand(B, S2, generator=g) + 0.5
    got = ref.indexer_logits(q, k, w, sc, sparse_mode=sparse_mode)
    want = _brute_logits(q, k, w, sc, sparse_mode)
    assert torch.equal(torch.isinf(got), torch.isinf(want))
    fin = torch.isfinite(want)
    torch.testing.assert_close(got[fin], want[fin], rtol=1e-5, atol=1e-5)


def test_indexer_logits_one_hot_probe_catches_transposes():
    # q nonzero only at (t=1, h=2, d=3); k only at (s=4, d=3): the single positive
    # logit must land at [t=1, s=4] and carry w[1, 2] * q * k * scale[4].
    B, S1, S2, H, D = 1, 3, 6, 4, 8
    q = torch.zeros(B, S1, H, D)
    k = torch.zeros(B, S2, D)
    q[0, 1, 2, 3] = 2.0
    k[0, 4, 3] = 3.0
    w = torch.zeros(B, S1, H)
    w[0, 1, 2] = 0.5
    sc = torch.arange(1, S2 + 1, dtype=torch.float32).view(1, S2)
    got = ref.indexer_logits(q, k, w, sc, sparse_mode=0)
    want = torch.zeros(B, S1, S2)
    want[0, 1, 4] = 0.5 * 6.0 * 5.0
    assert torch.equal(got, want)


def test_indexer_logits_linear_in_weights_and_homogeneous_in_scale():
    g = torch.Generator().manual_seed(2)
    B, S1, S2, H, D = 1, 8, 32, 16, 16
    q = torch.randn(B, S1, H, D, generator=g)
    k = torch.randn(B, S2, D, generator=g)
    w1 = torch.randn(B, S1, H, generator=g)
    w2 = torch.randn(B, S1, H, generator=g)
    sc = torch.rand(B, S2, generator=g) + 0.1
    a = ref.indexer_logits(q, k, w1 + w2, sc, sparse_mode=0)
    b = ref.indexer_logits(q, k, w1, sc, sparse_mode=0) + ref.indexer_logits(q, k, w2, sc, sparse_mode=0)
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)
    c = ref.indexer_logits(q, k, w1, 3.0 * sc, sparse_mode=0)
    torch.testing.assert_close(c, 3.0 * ref.indexer_logits(q, k, w1, sc, sparse_mode=0), rtol=1e-5, atol=1e-5)


def test_indexer_logits_one_hot_weight_is_relu_gemm():
    g = torch.Generator().manual_seed(3)
    B, S1, S2, H, D = 1, 5, 9, 4, 8
    q = torch.randn(B, S1, H, D, generator=g)
    k = torch.randn(B, S2, D, generator=g)
    w = torch.zeros(B, S1, H)
    w[..., 1] = 1.0
    got = ref.indexer_logits(q, k, w, sparse_mode=0)
    want = torch.relu(q[0, :, 1, :].double() @ k[0].double().T).float()
    torch.testing.assert_close(got[0], want, rtol=1e-6, atol=1e-6)


def test_indexer_causal_row_lengths():
    B, S1, S2 = 1, 4, 10
    out = ref.indexer_logits(torch.ones(B, S1, 16, 8), torch.ones(B, S2, 8), torch.ones(B, S1, 16), sparse_mode=3)
    finite = torch.isfinite(out[0]).sum(dim=1).tolist()
    assert finite == [S2 - S1 + t + 1 for t in range(S1)]


# --------------------------------------------------------------------------- sparse MLA
def _mla_inputs(B=1, S=6, Skv=64, H=16, topk=16, seed=5):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S, H, 576, generator=g) * 0.5
    kv = torch.randn(B, Skv, 1, 576, generator=g) * 0.5
    idx = ref.causal_sparse_indices(B, S, Skv, topk, seed=seed)
    return q, kv, idx


def test_mla_gather_equals_dense_mask_restatement():
    q, kv, idx = _mla_inputs()
    idx[0, 2, 0, 5:] = -1  # padded slots drop out
    out, _ = ref.sparse_mla_fwd(q, kv, idx)
    dense = ref.sparse_mla_dense_ref(q, kv, idx)
    torch.testing.assert_close(out, dense, rtol=1e-5, atol=1e-5)


def test_mla_skv_padding_equals_dense_golden():
    """The SFA example pads index lists with SKV, not -1 (example_sparse_flash_attn.py:303-308);
    its golden scatters them into an extra mask column that is cut off (:277-278).  The gather
    oracle drops indices >= kv_len the same way, with the golden's causal origin q_start."""
    q, kv, _ = _mla_inputs(S=4, Skv=96, topk=24)
    Skv, q_start = 96, 40
    g = torch.Generator().manual_seed(8)
    idx = torch.full((1, 4, 1, 24), Skv, dtype=torch.int32)
    for t in range(4):
        i_i = torch.randperm(t + q_start, generator=g)[:20]
        idx[0, t, 0, :len(i_i)] = i_i.to(torch.int32)
    dense = ref.sparse_mla_dense_ref(q, kv, idx, q_start_index_s=q_start)
    # The gather form's causal rule is idx <= kv_len - q_len + t: rows t see q_start + t.
    out, _ = ref.sparse_mla_fwd(q, kv[:, :q_start + 4], idx, actual_seq_lengths_kv=[q_start + 4])
    torch.testing.assert_close(out, dense, rtol=1e-5, atol=1e-5)
    # SKV slots are dropped: the same as -1 padding.
    out_m1, _ = ref.sparse_mla_fwd(q, kv[:, :q_start + 4], torch.where(idx == Skv, -1, idx),
                                   actual_seq_lengths_kv=[q_start + 4])
    torch.testing.assert_close(out, out_m1, rtol=0, atol=0)


def test_mla_single_index_closed_form():
    q, kv, _ = _mla_inputs(S=1)
    idx = torch.full((1, 1, 1, 8), -1, dtype=torch.int32)
    idx[0, 0, 0, 3] = 17
    out, lse = ref.sparse_mla_fwd(q, kv, idx)
    torch.testing.assert_close(out[0, 0], kv[0, 17, 0, :512].expand(16, 512), rtol=1e-6, atol=1e-6)
    want = (q[0, 0].double() @ kv[0, 17, 0].double()) / math.sqrt(576)
    torch.testing.assert_close(lse[0, 0].double(), want, rtol=1e-6, atol=1e-6)


def test_mla_equal_scores_give_mean_and_log_n():
    B, S, Skv, H, topk = 1, 1, 32, 16, 8
    q = torch.zeros(B, S, H, 576)
    kv = torch.randn(B, Skv, 1, 576)
    idx = torch.arange(topk, dtype=torch.int32).view(1, 1, 1, topk)
    out, lse = ref.sparse_mla_fwd(q, kv, idx)
    torch.testing.assert_close(out[0, 0], kv[0, :topk, 0, :512].mean(0).expand(H, 512), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(lse, torch.full((1, 1, H), math.log(topk)), rtol=1e-6, atol=1e-6)


def test_mla_permutation_invariance_and_lse():
    q, kv, idx = _mla_inputs(S=3, topk=32)
    out, lse = ref.sparse_mla_fwd(q, kv, idx)
    perm = torch.randperm(32, generator=torch.Generator().manual_seed(9))
    out2, lse2 = ref.sparse_mla_fwd(q, kv, idx[..., perm].contiguous())
    torch.testing.assert_close(out, out2, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(lse, lse2, rtol=1e-6, atol=1e-6)
    # LSE against torch.logsumexp on the gathered scores of one row.
    rows = idx[0, 1, 0].long()
    sc = (q[0, 1].double() @ kv[0, rows, 0].double().T) / math.sqrt(576)
    torch.testing.assert_close(lse[0, 1].double(), torch.logsumexp(sc, dim=1), rtol=1e-6, atol=1e-6)


def test_mla_paged_equals_contiguous():
    q, kv, idx = _mla_inputs(B=2, S=4, Skv=64, topk=16)
    bs = 8
    nblk = 64 // bs
    perm = torch.randperm(2 * nblk, generator=torch.Generator().manual_seed(4))
    pool = torch.empty(2 * nblk, bs, 1, 576)
    table = perm.view(2, nblk).to(torch.int32)
    for b in range(2):
        for j in range(nblk):
            pool[table[b, j]] = kv[b, j * bs:(j + 1) * bs]
    o1, l1 = ref.sparse_mla_fwd(q, kv, idx)
    o2, l2 = ref.sparse_mla_fwd(q, pool, idx, block_table=table)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_mla_causal_mask_drops_future_indices():
    q, kv, _ = _mla_inputs(S=4, Skv=16, topk=4)
    idx = torch.tensor([[[[0, 15, 3, -1]], [[1, 2, 14, 13]], [[5, 6, 7, 8]], [[15, 14, 0, 1]]]], dtype=torch.int32)
    out, lse = ref.sparse_mla_fwd(q, kv, idx)
    # Row s may use indices <= Skv - S + s = 12 + s.
    kept = torch.tensor([[[[0, -1, 3, -1]], [[1, 2, -1, 13]], [[5, 6, 7, 8]], [[15, 14, 0, 1]]]], dtype=torch.int32)
    out2, lse2 = ref.sparse_mla_fwd(q, kv, kept, is_causal=False)
    assert torch.equal(out, out2) and torch.equal(lse, lse2)


def test_mla_empty_row():
    q, kv, _ = _mla_inputs(S=1)
    idx = torch.full((1, 1, 1, 4), -1, dtype=torch.int32)
    out, lse = ref.sparse_mla_fwd(q, kv, idx)
    assert torch.all(out == 0) and torch.all(torch.isneginf(lse))


def test_causal_sparse_indices_are_unique_and_in_range():
    idx = ref.causal_sparse_indices(1, 64, 256, 128, seed=1)
    for t in range(64):
        row = idx[0, t, 0]
        valid = row[row >= 0]
        assert valid.numel() == min(128, 256 - 64 + t + 1)
        assert torch.unique(valid).numel() == valid.numel()
        assert int(valid.max()) <= 256 - 64 + t
        assert torch.all(row[valid.numel():] == -1)


def test_tnd_row_map_hand_worked():
    # Prefix sums [2, 2, 5]: lengths [2, 0, 3]; packed rows 0,1 -> batch 0, rows 2..4 -> batch 2.
    x = torch.tensor([[1.0], [2.0], [3.0], [4.0], [5.0]])
    padded, lens = ref.tnd_to_padded(x, [2, 2, 5])
    assert lens == [2, 0, 3]
    assert torch.equal(padded[..., 0], torch.tensor([[1.0, 2.0, 0.0], [0.0, 0.0, 0.0], [3.0, 4.0, 5.0]]))
    assert torch.equal(ref.padded_to_tnd(padded, lens), x)
    # Uniform lengths: packing is a reshape.
    y = torch.randn(12, 3, 4)
    p2, l2 = ref.tnd_to_padded(y, [4, 8, 12])
    assert l2 == [4, 4, 4] and torch.equal(p2, y.view(3, 4, 3, 4))


def test_tnd_indexer_equals_per_batch_bsnd():
    # Each batch of a ragged packed call equals a one-batch BSND call on its own rows.
    g = torch.Generator().manual_seed(5)
    q_lens, k_lens = [3, 0, 5], [9, 4, 12]
    H, D, K = 2, 8, 6
    q = torch.randn(sum(q_lens), H, D, generator=g)
    k = torch.randn(sum(k_lens), D, generator=g)
    w = torch.randn(sum(q_lens), H, generator=g)
    cu_q = list(np.cumsum(q_lens))
    cu_k = list(np.cumsum(k_lens))
    idx, val, logits = ref.lightning_indexer_tnd(q, k, w, cu_q, cu_k=cu_k, sparse_count=K, sparse_mode=3)
    assert idx.shape == (sum(q_lens), 1, K) and logits.shape == (sum(q_lens), max(k_lens))
    q0 = k0 = 0
    for aq, ak in zip(q_lens, k_lens):
        if aq:
            bi, bv, bl = ref.lightning_indexer(q[q0:q0 + aq][None], k[k0:k0 + ak][None], w[q0:q0 + aq][None],
                                               sparse_count=K, sparse_mode=3)
            assert torch.equal(idx[q0:q0 + aq], bi[0])
            assert torch.equal(logits[q0:q0 + aq, :ak], bl[0])
            assert torch.all(torch.isneginf(logits[q0:q0 + aq, ak:]))
        q0, k0 = q0 + aq, k0 + ak


def test_v4_slots_hand_worked():
    # Window clipped at 0; win_left = 127.
    o, c = ref.v4_slots(3, win_left=127)
    assert o == [0, 1, 2, 3] and c == []
    o, c = ref.v4_slots(300, win_left=127)
    assert o == list(range(173, 301))
    # hca: threshold floor((9 + 1) / 4) = 2.
    assert ref.v4_slots(9, win_left=2, cmp_ratio=4, dense_cmp=True) == ([7, 8, 9], [0, 1])
    # csa: threshold 3, only the first 3 entries are read; 5 >= 3 skipped, -1 ends the list.
    assert ref.v4_slots(11, win_left=0, cmp_ratio=4, sel=[5, 1, -1, 0]) == ([11], [1])
    assert ref.v4_slots(11, win_left=0, cmp_ratio=4, sel=[2, 0, 1, 0]) == ([11], [2, 0, 1])
    # Rows before the cache start see nothing.
    assert ref.v4_slots(-1, win_left=127, cmp_ratio=4, dense_cmp=True) == ([], [])


def _v4_one_batch(q, rows_ori, sinks, scale, win_left=127):
    """One batch, identity block table, a single query row at the end of the sequence."""
    T, H, D = q.shape
    n = rows_ori.shape[0]
    pool = rows_ori.view(n, 1, 1, D)
    table = torch.arange(n, dtype=torch.int32).view(1, n)
    return ref.sparse_flash_mla(q, [0, T], [n], pool, table, sinks, scale, ori_win_left=win_left)


def test_v4_sink_single_key_closed_form():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 2, 8, generator=g, dtype=torch.float64).float()
    k = torch.randn(1, 8, generator=g, dtype=torch.float64).float()
    sinks = torch.tensor([0.5, -1.0])
    out, lse = _v4_one_batch(q, k, sinks, 0.3)
    s = (q[0].double() @ k[0].double()) * 0.3
    w = torch.exp(s) / (torch.exp(s) + torch.exp(sinks.double()))
    assert torch.allclose(out[0].double(), w.view(2, 1) * k.double(), rtol=1e-6, atol=1e-6)
    assert torch.allclose(lse[0].double(), torch.log(torch.exp(s) + torch.exp(sinks.double())), rtol=1e-6)


def test_v4_sink_matches_library_softmax_and_vanishes():
    g = torch.Generator().manual_seed(4)
    H, D, n = 4, 16, 40
    q = torch.randn(1, H, D, generator=g)
    k = torch.randn(n, D, generator=g)
    sinks = torch.randn(H, generator=g)
    out, lse = _v4_one_batch(q, k, sinks, 0.25, win_left=31)
    keys = k[n - 32:].double()                       # window of 32 rows ending at the row's position
    sc = (q[0].double() @ keys.T) * 0.25
    full = torch.cat([sc, sinks.double().view(H, 1)], dim=1)
    p = torch.softmax(full, dim=1)[:, :-1]
    assert torch.allclose(out[0].double(), p @ keys, rtol=1e-5, atol=1e-6)
    assert torch.allclose(lse[0].double(), torch.logsumexp(full, dim=1), rtol=1e-6)
    # A sink far below every score leaves plain softmax attention.
    out2, lse2 = _v4_one_batch(q, k, torch.full((H,), -1e4), 0.25, win_left=31)
    p2 = torch.softmax(sc, dim=1)
    assert torch.allclose(out2[0].double(), p2 @ keys, rtol=1e-5, atol=1e-6)
    assert torch.allclose(lse2[0].double(), torch.logsumexp(sc, dim=1), rtol=1e-6)


def test_v4_golden_mode_matches_exact_without_rounding():
    # The golden-arithmetic mode with float32 P is the exact result up to float32 rounding.
    g = torch.Generator().manual_seed(6)
    H, D, n = 4, 32, 700
    q = torch.randn(3, H, D, generator=g)
    k = torch.randn(n, D, generator=g)
    sinks = torch.randn(H, generator=g)
    pool, table = k.view(n, 1, 1, D), torch.arange(n, dtype=torch.int32).view(1, n)
    ex = ref.sparse_flash_mla(q, [0, 3], [n], pool, table, sinks, 0.2, ori_win_left=600)
    gm = ref.sparse_flash_mla(q, [0, 3], [n], pool, table, sinks, 0.2, ori_win_left=600,
                              golden_p_dtype=torch.float32)
    assert torch.allclose(ex[0], gm[0], rtol=1e-4, atol=1e-5) and torch.allclose(ex[1], gm[1], rtol=1e-5)
    # bf16 P: the golden's own deviation from exact, small but nonzero.
    gb = ref.sparse_flash_mla(q, [0, 3], [n], pool, table, sinks, 0.2, ori_win_left=600,
                              golden_p_dtype=torch.bfloat16)
    d = (gb[0] - ex[0]).abs().max().item()
    assert 0 < d < 2e-2


def _scatter_to_pool(contig, bs, g):
    """Lay per-batch contiguous caches [B, L, D] out as a pool of blocks [B * L / bs, bs, 1, D] under
    a random permutation: block e of batch b goes to pool block table[b, e]."""
    B, L, D = contig.shape
    nb = L // bs
    perm = torch.randperm(B * nb, generator=g)
    table = perm.view(B, nb).to(torch.int32)
    pool = torch.empty(B * nb, bs, 1, D, dtype=contig.dtype)
    for b in range(B):
        for e in range(nb):
            pool[int(table[b, e])] = contig[b, e * bs:(e + 1) * bs].view(bs, 1, D)
    return pool, table


def test_unpack_paged_permuted_table_equals_contiguous_cache():
    g = torch.Generator().manual_seed(12)
    B, L, D, bs = 3, 96, 8, 16
    contig = torch.randn(B, L, D, generator=g)
    pool, table = _scatter_to_pool(contig, bs, g)
    assert not torch.equal(table.view(-1), torch.arange(B * L // bs, dtype=torch.int32))
    for b in range(B):
        for length in (L, 50, 16, 1):  # whole blocks and a partial last block
            assert torch.equal(ref.unpack_paged(pool, table, length, b), contig[b, :length])


def test_v4_paged_permuted_table_equals_contiguous_layout():
    # The whole V4 oracle on a permuted pool gives what it gives on the identity layout of the
    # same per-batch caches (original and compressed rows both paged).
    g = torch.Generator().manual_seed(13)
    B, L, D, bs, H, ratio = 2, 128, 16, 16, 4, 4
    ori = torch.randn(B, L, D, generator=g)
    cmp = torch.randn(B, L // ratio, D, generator=g)
    q = torch.randn(6, H, D, generator=g)
    sinks = torch.randn(H, generator=g)
    cu, kv_len = [0, 2, 6], [100, 128]
    pool_o, tab_o = _scatter_to_pool(ori, bs, g)
    pool_c, tab_c = _scatter_to_pool(cmp, bs // ratio, g)
    ident_o = torch.arange(B * L // bs, dtype=torch.int32).view(B, -1)
    ident_c = torch.arange(B * L // bs, dtype=torch.int32).view(B, -1)
    lin_o = ori.reshape(B * L // bs, bs, 1, D)
    lin_c = cmp.reshape(B * L // bs, bs // ratio, 1, D)
    a = ref.sparse_flash_mla(q, cu, kv_len, pool_o, tab_o, sinks, 0.3, cmp_kv=pool_c, cmp_block_table=tab_c,
                             cmp_ratio=ratio, ori_win_left=31)
    b = ref.sparse_flash_mla(q, cu, kv_len, lin_o, ident_o, sinks, 0.3, cmp_kv=lin_c, cmp_block_table=ident_c,
                             cmp_ratio=ratio, ori_win_left=31)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    # And a wrong table (the permutation's inverse) changes the result.
    inv = torch.argsort(tab_o.view(-1).long()).to(torch.int32).view(B, -1)
    c = ref.sparse_flash_mla(q, cu, kv_len, pool_o, inv, sinks, 0.3, cmp_kv=pool_c, cmp_block_table=tab_c,
                             cmp_ratio=ratio, ori_win_left=31)
    assert not torch.equal(a[0], c[0])


# ----------------------------------------------------- V4 sparse_attn with sinks
def test_sparse_attn_sink_one_key_closed_form():
    # Every slot on one key j: p is uniform over the K slots, so
    # out = kv[j] * K e^s / (K e^s + e^sink) and lse = log(K e^s + e^sink).
    g = torch.Generator().manual_seed(21)
    H, D, n, K = 3, 8, 5, 6
    q = torch.randn(1, 1, H, D, generator=g, dtype=torch.float64).float()
    kv = torch.randn(1, n, D, generator=g, dtype=torch.float64).float()
    sink = torch.tensor([0.3, -2.0, 1.5])
    idx = torch.full((1, 1, K), 2, dtype=torch.int32)
    out, lse = ref.sparse_attn_sink(q, kv, sink, idx, 0.4)
    s = (q[0, 0].double() @ kv[0, 2].double()) * 0.4
    z = K * torch.exp(s) + torch.exp(sink.double())
    w = K * torch.exp(s) / z
    assert torch.allclose(out[0, 0].double(), w.view(H, 1) * kv[0, 2].double(), rtol=1e-6, atol=1e-7)
    assert torch.allclose(lse[0, 0].double(), torch.log(z), rtol=1e-6)


def test_sparse_attn_sink_identity_against_plain_mla():
    # With a sink, out = out_plain * sigmoid(lse_plain - sink) and
    # lse = logaddexp(lse_plain, sink), where (out_plain, lse_plain) is the
    # separately pinned sparse_mla_fwd over the same unique slots (no causal mask).
    g = torch.Generator().manual_seed(22)
    B, M, H, D, n, K = 2, 3, 4, 16, 30, 10
    q = torch.randn(B, M, H, D, generator=g)
    kv = torch.randn(B, n, D, generator=g)
    sink = torch.randn(H, generator=g)
    idx = torch.stack([torch.randperm(n, generator=g)[:K] for _ in range(B * M)]).view(B, M, K).int()
    out, lse = ref.sparse_attn_sink(q, kv, sink, idx, 0.3)
    op, lp = ref.sparse_mla_fwd(q, kv.view(B, n, 1, D), idx.view(B, M, 1, K), 0.3, d_v=D, is_causal=False)
    f = torch.sigmoid(lp.double() - sink.double().view(1, 1, H)).unsqueeze(-1)
    assert torch.allclose(out.double(), op.double() * f, rtol=1e-5, atol=1e-6)
    assert torch.allclose(lse.double(), torch.logaddexp(lp.double(), sink.double().view(1, 1, H)), rtol=1e-6)
    # No sink: exactly the plain attention.
    o0, l0 = ref.sparse_attn_sink(q, kv, None, idx, 0.3)
    assert torch.allclose(o0, op, rtol=1e-5, atol=1e-6) and torch.allclose(l0, lp, rtol=1e-6)


def test_sparse_attn_sink_masked_and_duplicate_slots():
    g = torch.Generator().manual_seed(23)
    H, D, n = 2, 8, 12
    q = torch.randn(1, 1, H, D, generator=g)
    kv = torch.randn(1, n, D, generator=g)
    sink = torch.randn(H, generator=g)
    a = torch.tensor([[[3, -1, 7, -1, 0]]], dtype=torch.int32)
    b = torch.tensor([[[3, 7, 0]]], dtype=torch.int32)
    oa, la = ref.sparse_attn_sink(q, kv, sink, a, 0.5)
    ob, lb = ref.sparse_attn_sink(q, kv, sink, b, 0.5)
    assert torch.equal(oa, ob) and torch.equal(la, lb)           # -1 slots drop out
    # A key listed twice weighs twice: brute force with torch.softmax, sink appended.
    d = torch.tensor([[[3, 3, 7]]], dtype=torch.int32)
    od, ld = ref.sparse_attn_sink(q, kv, sink, d, 0.5)
    keys = kv[0, [3, 3, 7]].double()
    full = torch.cat([(q[0, 0].double() @ keys.T) * 0.5, sink.double().view(H, 1)], dim=1)
    p = torch.softmax(full, dim=1)[:, :-1]
    assert torch.allclose(od[0, 0].double(), p @ keys, rtol=1e-6, atol=1e-7)
    assert torch.allclose(ld[0, 0].double(), torch.logsumexp(full, dim=1), rtol=1e-6)
    # No valid slot: out 0, lse = sink.
    oe, le = ref.sparse_attn_sink(q, kv, sink, torch.full((1, 1, 4), -1, dtype=torch.int32), 0.5)
    assert torch.count_nonzero(oe) == 0 and torch.allclose(le[0, 0], sink)


def test_act_quant_int8_hand_worked():
    # amax 127 -> scale exactly 1: half-way values go to the even integer.
    x = torch.tensor([[127.0, 63.5, 62.5, -0.5, 0.5, 1.5, -2.5, -127.0]])
    y, s = ref.act_quant(x)
    assert s.item() == 1.0
    assert y[0].tolist() == [127, 64, 62, 0, 0, 2, -2, -127]
    # An all-zero row: the 1e-4 floor, y = 0.
    y0, s0 = ref.act_quant(torch.zeros(1, 8))
    assert torch.all(y0 == 0) and abs(s0.item() - 1e-4 / 127) < 1e-12
    # round_scale: power-of-two scale at or above amax / 127.
    g = torch.Generator().manual_seed(1)
    xr = torch.randn(16, 64, generator=g)
    _, sr = ref.act_quant(xr, round_scale=True)
    m = torch.log2(sr)
    assert torch.equal(m, torch.round(m)) and torch.all(sr >= xr.abs().amax(1, keepdim=True) / 127)
    assert torch.all(sr < 2 * xr.abs().amax(1, keepdim=True) / 127)
    # Error bound.
    yq, sq = ref.act_quant(xr)
    assert torch.all((xr - yq.float() * sq).abs() <= sq / 2 + 1e-7)


def test_act_quant_fp8_grid():
    # Row max 448 -> scale 1; e4m3 grid points stay, midpoints go to the even neighbour.
    x = torch.tensor([[448.0, 1.0, 1.125, 1.0625, 1.1875, -3.5, 0.001953125, 0.0029296875]])
    y, s = ref.act_quant(x, dtype=torch.float8_e4m3fn)
    assert s.item() == 1.0
    got = y.float()[0].tolist()
    # 1.0625 is the midpoint of 1.0 and 1.125 (mantissa 000 / 001): even -> 1.0;
    # 1.1875 is the midpoint of 1.125 and 1.25 (001 / 010): even -> 1.25;
    # 2^-9 is the smallest subnormal; 1.5 * 2^-9 is a midpoint -> 2 * 2^-9 (even).
    assert got == [448.0, 1.0, 1.125, 1.0, 1.25, -3.5, 0.001953125, 0.00390625]


# --------------------------------------------------------------------------- KV groups
def _gqa_inputs(B=2, S=5, Skv=23, G=3, Hg=2, D=16, topk=7, seed=11):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S, G * Hg, D, generator=g)
    kv = torch.randn(B, Skv, G, D, generator=g)
    idx = torch.full((B, S, G, topk), -1, dtype=torch.int32)
    for b in range(B):
        for t in range(S):
            for k in range(G):
                # Some slots past the causal bound (Skv - S + t) and some -1 padding.
                n = int(torch.randint(1, topk + 1, (1,), generator=g))
                sel = torch.randperm(Skv, generator=g)[:n]
                idx[b, t, k, :n] = sel.to(torch.int32)
    return q, kv, idx


@pytest.mark.parametrize("D,d_v", [(16, 16), (24, 16)])
def test_grouped_gather_equals_dense_gqa_golden(D, d_v):
    q, kv, idx = _gqa_inputs(D=D)
    out, _ = ref.sparse_attention_grouped(q, kv, idx, d_v=d_v)
    dense = ref.sparse_gqa_dense_ref(q, kv, idx, d_v=d_v)
    torch.testing.assert_close(out, dense, rtol=1e-5, atol=1e-5)
    # A head-to-group map by interleaving (h % G) instead of blocks would differ.
    perm = torch.arange(q.shape[2]).view(2, 3).t().reshape(-1)
    wrong, _ = ref.sparse_attention_grouped(q[:, :, perm], kv, idx, d_v=d_v)
    assert (wrong[:, :, perm.argsort()] - dense).abs().max() > 1e-2


def test_grouped_one_group_equals_sparse_mla_fwd():
    q, kv, idx = _mla_inputs()
    out_g, lse_g = ref.sparse_attention_grouped(q, kv, idx, d_v=512)
    out, lse = ref.sparse_mla_fwd(q, kv, idx)
    torch.testing.assert_close(out_g, out, rtol=0, atol=0)
    torch.testing.assert_close(lse_g, lse, rtol=0, atol=0)


def test_grouped_permuting_groups_permutes_outputs():
    q, kv, idx = _gqa_inputs()
    out, lse = ref.sparse_attention_grouped(q, kv, idx, d_v=16)
    gp = torch.tensor([2, 0, 1])
    hp = torch.cat([torch.arange(2) + 2 * int(k) for k in gp])
    out_p, lse_p = ref.sparse_attention_grouped(q[:, :, hp], kv[:, :, gp], idx[:, :, gp], d_v=16)
    torch.testing.assert_close(out_p, out[:, :, hp], rtol=0, atol=0)
    torch.testing.assert_close(lse_p, lse[:, :, hp], rtol=0, atol=0)


def test_grouped_single_index_per_group_closed_form():
    q, kv, _ = _gqa_inputs(B=1, S=1)
    idx = torch.full((1, 1, 3, 7), -1, dtype=torch.int32)
    picks = [4, 9, 17]
    for k, j in enumerate(picks):
        idx[0, 0, k, 5] = j
    out, lse = ref.sparse_attention_grouped(q, kv, idx, d_v=16)
    for k, j in enumerate(picks):
        torch.testing.assert_close(out[0, 0, 2 * k:2 * k + 2], kv[0, j, k].expand(2, 16), rtol=1e-6, atol=1e-6)
        want = (q[0, 0, 2 * k:2 * k + 2].double() @ kv[0, j, k].double()) / 4.0
        torch.testing.assert_close(lse[0, 0, 2 * k:2 * k + 2].double(), want, rtol=1e-6, atol=1e-6)
