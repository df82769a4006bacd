"""Child process of tests/test_zz_no_alloc.py::test_noalloc_first_call_inside_graph_capture.

In a fresh process (so the library has not yet looked up its scratch array on this device), one
eager call of the workspace entry dsa_sparse_mla_fwd warms the library up, as graph warm-up does;
then the process's first dsa_sparse_mla_fwd_noalloc call -- whose first step on a device is the
scratch lookup -- runs inside torch.cuda.graph capture, on a decode shape whose split partials live
in the scratch.  The graph is replayed three times, with eager work and host syncs between the
replays, and every replay must equal the workspace entry bit for bit.  Prints "ok" on success.
"""
import sys
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def main():
    import __graft_entry__

    pkg = __graft_entry__.load_package()
    lib = pkg.load_library()
    from tilelang_ascend_amd import _lib as L

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator().manual_seed(5)
    B, H, topk, ctx, bs = 3, 64, 512, 2048, 32
    nblk = ctx // bs
    q = (torch.randn(B, 1, H, 576, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    pool = (torch.randn(B * nblk, bs, 1, 576, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    table = torch.randperm(B * nblk, generator=g).view(B, nblk).to(torch.int32).to(dev)
    idx = torch.stack([torch.randperm(ctx, generator=g)[:topk] for _ in range(B)]).to(torch.int32)
    idx = idx.view(B, 1, 1, topk).to(dev)
    kl = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    need = lib.dsa_sparse_mla_workspace_size(B, 1, H, topk)
    assert 0 < need <= lib.dsa_sparse_mla_noalloc_max_workspace(), need

    def args(out, lse):
        return (L.KIND_BF16, q.data_ptr(), pool.data_ptr(), idx.data_ptr(), table.data_ptr(), None, kl.data_ptr(),
                B, 1, H, 576, 512, ctx, bs, nblk, topk, 576 ** -0.5, 1, out.data_ptr(), lse.data_ptr())

    want_o = torch.empty(B, 1, H, 512, dtype=torch.bfloat16, device=dev)
    want_l = torch.empty(B, 1, H, dtype=torch.float32, device=dev)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    L.check(lib.dsa_sparse_mla_fwd(*args(want_o, want_l), ws.data_ptr(), need, L.stream_handle(dev)), "eager")
    torch.cuda.synchronize()

    out = torch.empty_like(want_o)
    lse = torch.empty_like(want_l)
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            rc = lib.dsa_sparse_mla_fwd_noalloc(*args(out, lse), L.stream_handle(dev))
    torch.cuda.current_stream().wait_stream(s)
    assert rc == 0, lib.dsa_last_error_message()
    for rep in range(3):
        out.fill_(float("nan"))
        lse.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want_o) and torch.equal(lse, want_l), f"replay {rep}"
        # Eager work between replays: the same call, eagerly, on the shared scratch.
        L.check(lib.dsa_sparse_mla_fwd_noalloc(*args(want_o, want_l), L.stream_handle(dev)), "eager noalloc")
        torch.cuda.synchronize()
    print("ok", flush=True)


if __name__ == "__main__":
    main()
