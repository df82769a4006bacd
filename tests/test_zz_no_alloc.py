"""dsa_sparse_mla_fwd_noalloc (the allocation-free sparse MLA entry, split partials in a
library-owned per-GPU scratch array) against dsa_sparse_mla_fwd with a caller workspace,
through the C ABI: bit-equal outputs on two calls in a row (the second smaller), a call with
no split (no scratch used), the rejection of a shape whose partials exceed the scratch, and a
process's first noalloc call (the scratch lookup) made inside HIP-graph capture."""
import subprocess
import sys
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu


def _decode_inputs(dev, B, H, topk, ctx, bs, seed):
    g = torch.Generator().manual_seed(seed)
    nblk = ctx // bs
    q = (torch.randn(B, 1, H, 576, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    pool = (torch.randn(B * nblk, bs, 1, 576, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    table = torch.randperm(B * nblk, generator=g).view(B, nblk).to(torch.int32).to(dev)
    idx = torch.stack([torch.randperm(ctx, generator=g)[:topk] for _ in range(B)]).to(torch.int32)
    idx[0, 5:17] = -1                                    # a few empty slots
    lens = torch.full((B,), ctx, dtype=torch.int32)
    return q, pool, table, idx.view(B, 1, 1, topk).to(dev), lens.to(dev), torch.ones(B, dtype=torch.int32).to(dev)


def _run(dsa, L, lib, dev, q, pool, table, idx, kl, ql, noalloc):
    B, S, H, _ = q.shape
    bs, nblk, topk = pool.shape[1], table.shape[1], idx.shape[-1]
    out = torch.full((B, S, H, 512), float("nan"), dtype=torch.bfloat16, device=dev)
    lse = torch.full((B, S, H), float("nan"), dtype=torch.float32, device=dev)
    args = (L.KIND_BF16, q.data_ptr(), pool.data_ptr(), idx.data_ptr(), table.data_ptr(), ql.data_ptr(),
            kl.data_ptr(), B, S, H, 576, 512, nblk * bs, bs, nblk, topk, 576 ** -0.5, 1, out.data_ptr(),
            lse.data_ptr())
    stream = L.stream_handle(dev)
    if noalloc:
        L.check(lib.dsa_sparse_mla_fwd_noalloc(*args, stream), "noalloc")
    else:
        need = lib.dsa_sparse_mla_workspace_size(B, S, H, topk)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        L.check(lib.dsa_sparse_mla_fwd(*args, ws.data_ptr(), need, stream), "workspace")
    torch.cuda.synchronize()
    return out, lse


def test_noalloc_equals_workspace_entry(dsa, dev):
    from tilelang_ascend_amd import _lib as L

    lib = dsa.load_library()
    assert lib.dsa_sparse_mla_noalloc_max_workspace() == 64 << 20
    # Two decode calls in a row on the shared scratch, the second smaller; then a prefill-shaped
    # call that takes no split (no scratch).
    cases = [dict(B=16, H=128, topk=2048, ctx=8192, bs=64, seed=1),
             dict(B=3, H=64, topk=512, ctx=2048, bs=32, seed=2),
             dict(B=300, H=16, topk=256, ctx=1024, bs=64, seed=3)]
    for n, c in enumerate(cases):
        print(f"noalloc case {n}: {c}", flush=True)
        t = _decode_inputs(dev, **c)
        need = lib.dsa_sparse_mla_workspace_size(c["B"], 1, c["H"], c["topk"])
        assert (need > 0) == (n < 2)
        want = _run(dsa, L, lib, dev, *t, noalloc=False)
        got = _run(dsa, L, lib, dev, *t, noalloc=True)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1]), f"case {n}"
        assert not torch.isnan(got[1]).any()


def test_noalloc_rejects_partials_beyond_the_scratch(dsa, dev):
    lib = dsa.load_library()
    # topk 4096 splits every row in two: 1000 tokens x 128 heads x 2 splits x 1028 B > 64 MiB.
    assert lib.dsa_sparse_mla_workspace_size(1, 1000, 128, 4096) > lib.dsa_sparse_mla_noalloc_max_workspace()
    x = torch.empty(16, device=dev)
    rc = lib.dsa_sparse_mla_fwd_noalloc(1, x.data_ptr(), x.data_ptr(), x.data_ptr(), None, None, None, 1, 1000, 128,
                                        576, 512, 4096, 0, 0, 4096, 0.04, 1, x.data_ptr(), x.data_ptr(), None)
    assert rc == 1 and b"scratch" in lib.dsa_last_error_message()


def test_noalloc_first_call_inside_graph_capture():
    """A fresh process warms up through the workspace entry, then makes its first noalloc call
    (the per-device scratch lookup included) inside torch.cuda.graph capture; three replays equal
    the workspace entry bit for bit (tests/noalloc_capture_child.py)."""
    child = Path(__file__).resolve().parent / "noalloc_capture_child.py"
    res = subprocess.run([sys.executable, str(child)], capture_output=True, text=True, timeout=240)
    assert res.returncode == 0 and res.stdout.strip().endswith("ok"), res.stdout[-2000:] + res.stderr[-2000:]
