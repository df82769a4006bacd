"""Writes the golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

Every expected output here comes from a closed form or a brute-force
pure-Python computation, not from the oracle under test:

* kat_sort_arange131.npz  -- the reference's sort KAT
  (testing/python/language/test_tilelang_ascend_language_elementwise.py:4030-4086):
  input arange(131), expected descending values and their indices.
* kat_topk_arange51_k10.npz -- the reference's top-k KAT (same file :4189-4248):
  input arange(51), K = 10.
* ties_topk.npz -- small integer-valued rows full of ties, -inf masks and a
  NaN, top-K by brute force: Python's stable sort on (-value) with masked /
  NaN entries excluded and -1 padding (the rule of
  examples/deepseek_v4/lightning_indexer.py:317-325).
"""
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def brute_topk(row, k):
    cand = [(float(v), i) for i, v in enumerate(row) if not np.isnan(v) and v > -1e30]
    cand.sort(key=lambda t: (-t[0], t[1]))  # value desc, index asc
    idx = [i for _, i in cand[:k]] + [-1] * max(0, k - len(cand))
    val = [v for v, _ in cand[:k]] + [float("-inf")] * max(0, k - len(cand))
    return idx, val


def main():
    a = np.arange(131, dtype=np.float32)
    np.savez(HERE / "kat_sort_arange131.npz", x=a[None, :], idx=np.arange(130, -1, -1, dtype=np.int32)[None, :],
             val=a[::-1].copy()[None, :])
    a = np.arange(51, dtype=np.float32)
    np.savez(HERE / "kat_topk_arange51_k10.npz", x=a[None, :], k=np.int32(10),
             idx=np.arange(50, 40, -1, dtype=np.int32)[None, :], val=np.arange(50, 40, -1, dtype=np.float32)[None, :])
    rng = np.random.default_rng(20261201)
    rows, n, k = 16, 300, 40
    x = rng.integers(0, 6, size=(rows, n)).astype(np.float32)
    x[1, :] = 2.0                      # constant row
    x[2, 250:] = -np.inf               # masked tail
    x[3, :] = -np.inf
    x[3, :7] = 1.0                     # fewer valid than k
    x[4, 5] = np.nan                   # NaN never selected
    x[5, ::2] = -0.0
    x[5, 1::2] = 0.0                   # signed zeros tie
    x[6, :] = -1e31                    # finite but <= -1e30: all -1
    idx = np.zeros((rows, k), np.int32)
    val = np.zeros((rows, k), np.float32)
    for r in range(rows):
        i, v = brute_topk(x[r], k)
        idx[r], val[r] = i, v
    np.savez(HERE / "ties_topk.npz", x=x, k=np.int32(k), idx=idx, val=val)


if __name__ == "__main__":
    main()
