"""GPU parity of the radix top-k selector against the CPU oracle (bit-exact indices)."""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as ref

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _check(dsa, dev, x, k, sorted=True, row_len=None):
    idx, val = dsa.topk_selector(x.to(dev), k, sorted=sorted, return_values=True,
                                 row_len=None if row_len is None else row_len.to(dev))
    torch.cuda.synchronize()
    ri, rv = ref.topk_stable(x, k, valid_len=None if row_len is None else row_len.tolist())
    idx, val = idx.cpu(), val.cpu()
    if sorted:
        assert torch.equal(idx, ri), f"first mismatching row {int((idx != ri).any(1).nonzero()[0])}"
        assert torch.equal(val, rv)
    else:
        for r in range(x.shape[0]):
            assert set(idx[r].tolist()) == set(ri[r].tolist()), f"row {r}"
    return idx


@pytest.mark.parametrize("name", ["kat_sort_arange131.npz", "kat_topk_arange51_k10.npz", "ties_topk.npz"])
def test_golden_fixtures(dsa, dev, name):
    d = np.load(GOLDEN / name)
    x = torch.from_numpy(d["x"])
    k = int(d["k"]) if "k" in d else x.shape[1]
    idx, val = dsa.topk_selector(x.to(dev), k, return_values=True)
    assert np.array_equal(idx.cpu().numpy(), d["idx"])
    assert np.array_equal(val.cpu().numpy(), d["val"])


@pytest.mark.parametrize("B,N,K", [(64, 4096, 2048), (1024, 1024, 128)])  # example_topk_selector.py:124-138
def test_reference_example_cases(dsa, dev, B, N, K):
    g = torch.Generator().manual_seed(0)
    _check(dsa, dev, torch.randn(B, N, generator=g), K)


@pytest.mark.parametrize("N", [32768, 131072])  # LDS-cached and streaming paths
def test_long_rows(dsa, dev, N):
    g = torch.Generator().manual_seed(N)
    _check(dsa, dev, torch.randn(6, N, generator=g) * 3.0, 2048)


def test_many_ties_quantised_scores(dsa, dev):
    g = torch.Generator().manual_seed(3)
    x = torch.randint(0, 16, (32, 5000), generator=g).float()
    _check(dsa, dev, x, 777)


def test_unsorted_mode_same_set(dsa, dev):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(16, 9000, generator=g)
    _check(dsa, dev, x, 2048, sorted=False)
    xt = torch.randint(0, 4, (8, 3000), generator=g).float()
    _check(dsa, dev, xt, 1000, sorted=False)


def test_row_len_and_padding(dsa, dev):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(8, 4096, generator=g)
    row_len = torch.tensor([0, 1, 100, 2047, 2048, 2049, 4000, 4096], dtype=torch.int32)
    _check(dsa, dev, x, 2048, row_len=row_len)


def test_causal_masked_rows(dsa, dev):
    g = torch.Generator().manual_seed(6)
    S, N = 64, 3000
    x = torch.randn(S, N, generator=g)
    for t in range(S):
        x[t, t * 40 + 1:] = float("-inf")
    _check(dsa, dev, x, 2048)


def test_odd_length_and_strided_rows(dsa, dev):
    g = torch.Generator().manual_seed(7)
    base = torch.randn(10, 1003, generator=g)
    _check(dsa, dev, base[:, :999], 64)  # ld=1003, unaligned rows
    _check(dsa, dev, base, 1003)         # k == n


def test_deterministic_repeat(dsa, dev):
    g = torch.Generator().manual_seed(8)
    x = torch.randint(0, 3, (16, 20000), generator=g).float().to(dev)
    a = dsa.topk_selector(x, 2048)
    b = dsa.topk_selector(x, 2048)
    c = dsa.topk_selector(x, 2048, sorted=False)
    d = dsa.topk_selector(x, 2048, sorted=False)
    assert torch.equal(a, b) and torch.equal(c, d)


def test_builder_signature(dsa, dev):
    g = torch.Generator().manual_seed(9)
    x = torch.randn(4, 2048, generator=g)
    kern = dsa.simple_topk_selector(4, 2048, 512, 128)
    got = kern(x.to(dev)).cpu()
    assert torch.equal(got, ref.topk_stable(x, 512)[0])


def test_mixed_fast_and_exact_rows(dsa, dev):
    # Rows the register fast path cannot bound (constant rows, few distinct values,
    # a huge outlier) go to the exact radix pass; the others must be left untouched.
    g = torch.Generator().manual_seed(10)
    x = torch.randn(12, 30000, generator=g)
    x[1] = 0.5
    x[4] = torch.randint(0, 3, (30000,), generator=g).float()
    x[7, 123] = 3.0e38
    x[7, 5000] = -3.0e38
    x[10, :] = float("-inf")
    x[10, 17] = 1.0
    _check(dsa, dev, x, 2048)
    _check(dsa, dev, x, 100, sorted=False)


@pytest.mark.parametrize("N", [4096, 32768])
def test_whole_rows_exact_in_place(dsa, dev, N):
    """Whole 16-byte aligned rows (4096 * chunks scores, no lengths): the rows the register path
    cannot bound take the exact select inside the same workgroup, with no pass behind."""
    g = torch.Generator().manual_seed(N + 11)
    x = torch.randn(10, N, generator=g)
    x[1] = 0.5                                                 # one value throughout
    x[3] = torch.randint(0, 3, (N,), generator=g).float()      # three values
    x[5, 123] = 3.0e38                                         # outliers
    x[5, N // 2] = -3.0e38
    x[7, :] = float("-inf")
    x[7, 17] = 1.0                                             # a single present score
    x[8, ::2] = 2.0                                            # ties on every other position
    _check(dsa, dev, x, 2048)
    _check(dsa, dev, x, 1, sorted=False)
    _check(dsa, dev, x, 4096)


# Rows longer than 32768 scores: segments, then a top-k over the segments' candidates.
@pytest.mark.parametrize("N,K", [(131072, 2048), (50001, 100), (40000, 4096)])
def test_long_rows_two_stage(dsa, dev, N, K):
    g = torch.Generator().manual_seed(N + K)
    x = torch.randn(5, N, generator=g)
    x[1, N // 2:] = float("-inf")                 # masked tail
    x[2, :] = float("-inf")
    x[2, 7] = 0.25                                # a single present score
    x[3] = torch.randint(0, 5, (N,), generator=g).float()  # heavy ties: exact fallback
    _check(dsa, dev, x, K)


def test_long_rows_row_len_and_strides(dsa, dev):
    g = torch.Generator().manual_seed(77)
    base = torch.randn(4, 70003, generator=g)
    x = base[:, :70000]                           # ld 70003: unaligned rows
    row_len = torch.tensor([70000, 65537, 2048, 0], dtype=torch.int32)
    _check(dsa, dev, x, 2048, row_len=row_len)


def test_row_len_aligned_rows_every_tail(dsa, dev):
    """16-byte aligned rows of 8 register chunks with row lengths: the last whole group of 4 in an
    even and an odd chunk, a partial group after it or none, lengths below 4 (no whole group)."""
    g = torch.Generator().manual_seed(78)
    x = torch.randn(14, 32768, generator=g)
    x[12, 9000:] = float("-inf")  # masked inside the length
    row_len = torch.tensor([0, 1, 3, 5, 2049, 4097, 8195, 16386, 20001, 28673, 32767, 32768, 30000, 4096],
                           dtype=torch.int32)
    _check(dsa, dev, x, 2048, row_len=row_len)
    _check(dsa, dev, x, 100, sorted=False, row_len=row_len)
    x2 = torch.randn(6, 20000, generator=g)  # 20000 scores a row: 8 chunks, the last ones past the row
    _check(dsa, dev, x2, 2048, row_len=torch.tensor([0, 2, 2050, 10001, 19999, 20000], dtype=torch.int32))
    _check(dsa, dev, x2, 2048)


def test_long_rows_ws_matches_plain_entry(dsa, dev):
    # dsa_topk_select (no workspace: radix passes) and dsa_topk_select_ws agree bit for bit.
    from tilelang_ascend_amd import _lib as L
    g = torch.Generator().manual_seed(78)
    x = (torch.randn(3, 100000, generator=g) * 4).to(dev)
    lib = L.load_library()
    a = torch.empty(3, 2048, dtype=torch.int32, device=dev)
    b = torch.empty_like(a)
    st = L.stream_handle(dev)
    L.check(lib.dsa_topk_select(x.data_ptr(), 100000, 3, 100000, 2048, None, 1, a.data_ptr(), None, st), "plain")
    nws = lib.dsa_topk_select_workspace_size(3, 100000, 2048)
    assert nws > 0
    ws = torch.empty(nws, dtype=torch.uint8, device=dev)
    L.check(lib.dsa_topk_select_ws(x.data_ptr(), 100000, 3, 100000, 2048, None, 1, b.data_ptr(), None,
                                   ws.data_ptr(), nws, st), "ws")
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_structured_rows_crowd_waves(dsa, dev):
    # Rows whose top scores sit in a few threads' registers: sorted rows, sorted
    # runs (the shape of the second stage over segment candidates), and a
    # pattern repeating every 4096 positions.  The fast path then compacts the
    # candidates densely instead of per wave; results stay exact.
    g = torch.Generator().manual_seed(91)
    n = 32768
    pos = torch.arange(n)
    rows = [
        pos.float(),                                            # ascending
        -pos.float(),                                           # descending
        torch.cat([torch.sort(torch.randn(n // 4, generator=g), descending=True).values for _ in range(4)]),
        torch.randn(n, generator=g) + 10.0 * ((pos % 4096) < 256).float(),
        torch.randn(n, generator=g) + 10.0 * ((pos % 4096) >= 3840).float(),
    ]
    _check(dsa, dev, torch.stack(rows), 2048)
    runs = torch.stack([torch.cat([torch.sort(torch.randn(2048, generator=g), descending=True).values
                                   for _ in range(4)]) for _ in range(6)])
    _check(dsa, dev, runs, 2048)                                # n = 8192: four sorted runs of 2048


def test_candidates_across_zero(dsa, dev):
    # Rows whose candidates straddle zero: the binning then collapses magnitudes
    # far below the largest one (the plain order key would crowd them into a few
    # bins).  Shifted Gaussians (k-th score negative), a huge outlier on either
    # side, signed zeros and denormals around zero, and a row whose largest
    # magnitude is itself a denormal (no collapse).
    g = torch.Generator().manual_seed(123)
    n = 32768
    rows = [torch.randn(n, generator=g) - s for s in (1.2, 1.6, 2.5)]
    r = torch.randn(n, generator=g) - 1.5
    r[77] = 1.0e30
    rows.append(r)
    r = torch.randn(n, generator=g) - 1.5
    r[5] = -3.0e38
    r[9] = 2.0e-3
    rows.append(r)
    r = torch.randn(n, generator=g) * 1e-3
    r[::7] = 0.0
    r[3::7] = -0.0
    r[1::11] = 1e-42
    r[2::13] = -1e-42
    rows.append(r)
    r = (torch.randn(n, generator=g).sign() * 1e-40).float()
    rows.append(r)
    x = torch.stack(rows)
    _check(dsa, dev, x, 2048)
    _check(dsa, dev, x, 333)
    _check(dsa, dev, x[:, :9000], 2048)
